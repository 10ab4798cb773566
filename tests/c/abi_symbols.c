/*
 * abi_symbols.c - include/llmr_hip.h compiled as strict C11 (-pedantic
 * -Werror) and linked against libllmr_hip.so: every entry point the header
 * declares is referenced here, so the link fails if one is missing. Run, it
 * prints the number of resolved entry points (no device is touched).
 */
#include <stdint.h>
#include <stdio.h>

#include "llmr_hip.h"

/* Function pointers pass through uintptr_t: ISO C has no conversion between
 * differently typed function pointers and void*. */
static const struct {
    const char* name;
    void (*fn)(void);
} entry_points[] = {
    {"llmr_create_context", (void (*)(void))(uintptr_t)llmr_create_context},
    {"llmr_destroy_context", (void (*)(void))(uintptr_t)llmr_destroy_context},
    {"llmr_set_stream", (void (*)(void))(uintptr_t)llmr_set_stream},
    {"llmr_get_stream", (void (*)(void))(uintptr_t)llmr_get_stream},
    {"llmr_last_error", (void (*)(void))(uintptr_t)llmr_last_error},
    {"llmr_alloc", (void (*)(void))(uintptr_t)llmr_alloc},
    {"llmr_free", (void (*)(void))(uintptr_t)llmr_free},
    {"llmr_upload", (void (*)(void))(uintptr_t)llmr_upload},
    {"llmr_download", (void (*)(void))(uintptr_t)llmr_download},
    {"llmr_sync", (void (*)(void))(uintptr_t)llmr_sync},
    {"llmr_ggml_row_bytes", (void (*)(void))(uintptr_t)llmr_ggml_row_bytes},
    {"llmr_dequant", (void (*)(void))(uintptr_t)llmr_dequant},
    {"llmr_dequant_operand_f16", (void (*)(void))(uintptr_t)llmr_dequant_operand_f16},
    {"llmr_batch_matmul", (void (*)(void))(uintptr_t)llmr_batch_matmul},
    {"llmr_batch_matmul_pc", (void (*)(void))(uintptr_t)llmr_batch_matmul_pc},
    {"llmr_batch_matmul_noalloc", (void (*)(void))(uintptr_t)llmr_batch_matmul_noalloc},
    {"llmr_batch_matmul_multi", (void (*)(void))(uintptr_t)llmr_batch_matmul_multi},
    {"llmr_flash_attention_rows", (void (*)(void))(uintptr_t)llmr_flash_attention_rows},
    {"llmr_batch_matmul_multi_images", (void (*)(void))(uintptr_t)llmr_batch_matmul_multi_images},
    {"llmr_batch_matmul_multi_qkv", (void (*)(void))(uintptr_t)llmr_batch_matmul_multi_qkv},
    {"llmr_weight_image_bytes", (void (*)(void))(uintptr_t)llmr_weight_image_bytes},
    {"llmr_swiglu_weight_image_bytes", (void (*)(void))(uintptr_t)llmr_swiglu_weight_image_bytes},
    {"llmr_batch_layernorm_split", (void (*)(void))(uintptr_t)llmr_batch_layernorm_split},
    {"llmr_gated_residual_rmsnorm", (void (*)(void))(uintptr_t)llmr_gated_residual_rmsnorm},
    {"llmr_build_weight_image", (void (*)(void))(uintptr_t)llmr_build_weight_image},
    {"llmr_batch_matmul_swiglu", (void (*)(void))(uintptr_t)llmr_batch_matmul_swiglu},
    {"llmr_batch_matmul_swiglu_pc", (void (*)(void))(uintptr_t)llmr_batch_matmul_swiglu_pc},
    {"llmr_gguf_open", (void (*)(void))(uintptr_t)llmr_gguf_open},
    {"llmr_gguf_close", (void (*)(void))(uintptr_t)llmr_gguf_close},
    {"llmr_gguf_info", (void (*)(void))(uintptr_t)llmr_gguf_info},
    {"llmr_gguf_tensor", (void (*)(void))(uintptr_t)llmr_gguf_tensor},
    {"llmr_gguf_find_tensor", (void (*)(void))(uintptr_t)llmr_gguf_find_tensor},
    {"llmr_gguf_kv", (void (*)(void))(uintptr_t)llmr_gguf_kv},
    {"llmr_gguf_find_kv", (void (*)(void))(uintptr_t)llmr_gguf_find_kv},
    {"llmr_gguf_upload_tensor", (void (*)(void))(uintptr_t)llmr_gguf_upload_tensor},
    {"llmr_gguf_load_tensor", (void (*)(void))(uintptr_t)llmr_gguf_load_tensor},
    {"llmr_lora_correction", (void (*)(void))(uintptr_t)llmr_lora_correction},
    {"llmr_batch_matmul_lora", (void (*)(void))(uintptr_t)llmr_batch_matmul_lora},
    {"llmr_q8_lora_merge", (void (*)(void))(uintptr_t)llmr_q8_lora_merge},
    {"llmr_flash_attention", (void (*)(void))(uintptr_t)llmr_flash_attention},
    {"llmr_flash_attention_pc", (void (*)(void))(uintptr_t)llmr_flash_attention_pc},
    {"llmr_batch_rmsnorm", (void (*)(void))(uintptr_t)llmr_batch_rmsnorm},
    {"llmr_batch_layernorm", (void (*)(void))(uintptr_t)llmr_batch_layernorm},
    {"llmr_qkv_heads", (void (*)(void))(uintptr_t)llmr_qkv_heads},
    {"llmr_gated_residual", (void (*)(void))(uintptr_t)llmr_gated_residual},
    {"llmr_activation", (void (*)(void))(uintptr_t)llmr_activation},
    {"llmr_timestep_embed", (void (*)(void))(uintptr_t)llmr_timestep_embed},
    {"llmr_patchify", (void (*)(void))(uintptr_t)llmr_patchify},
    {"llmr_unpatchify", (void (*)(void))(uintptr_t)llmr_unpatchify},
    {"llmr_synth_q4k", (void (*)(void))(uintptr_t)llmr_synth_q4k},
};

int main(void) {
    size_t n = sizeof entry_points / sizeof entry_points[0], resolved = 0;
    for (size_t i = 0; i < n; i++)
        if (entry_points[i].fn) resolved++;
    printf("%zu of %zu entry points resolved\n", resolved, n);
    return resolved == n ? 0 : 1;
}
