/*
 * zimage_layer.c - a plain C11 caller of the C-ABI (include/llmr_hip.h) that
 * replays the Z-Image transformer layer the way the reference's C3 host
 * issues it (dit_transformer_layer, dependencies/zimage.c3l/dit.c3:1372-1627):
 * f32 activation buffers throughout, each GEMM through llmr_batch_matmul_pc
 * with a filled-in BatchMatMulPC (dit.c3:172-178), the SwiGLU through
 * llmr_batch_matmul_swiglu_pc, attention through llmr_flash_attention_pc with
 * a FlashAttentionPC (dit.c3:136-142).
 *
 *   zimage_layer DIR DIM HEADS FFN SEQ
 *
 * reads DIR/{hidden,attn_norm1,attn_norm2,ffn_norm1,ffn_norm2,q_norm,k_norm,
 * adaln,rope_cos,rope_sin}.f32 and DIR/{wqkv,wo,w_gate,w_up,w_down}.q8
 * (raw GGUF Q8_0 blocks), runs the layer on device 0 and writes the updated
 * hidden state to DIR/out.f32. It also runs the three per-slot Q/K/V calls
 * of the reference (row_offset 0, dim, 2*dim, dit.c3:1437-1442) and checks
 * that they equal the fused call's column slots bit for bit. Exit status 0
 * when every call succeeded and the slots matched; a failing call prints
 * llmr_last_error().
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "llmr_hip.h"

static llmr_context* ctx;
static const char* dir;

#define CHECK(call)                                                                      \
    do {                                                                                 \
        int rc_ = (call);                                                                \
        if (rc_ != LLMR_OK) {                                                            \
            fprintf(stderr, "%s:%d: %s -> %d: %s\n", __FILE__, __LINE__, #call, rc_,     \
                    llmr_last_error());                                                  \
            exit(1);                                                                     \
        }                                                                                \
    } while (0)

/* Reads DIR/name into a new host buffer of exactly `bytes` bytes. */
static void* read_file(const char* name, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(1);
    }
    void* buf = malloc(bytes ? bytes : 1);
    size_t got = fread(buf, 1, bytes, f);
    int extra = fgetc(f);
    fclose(f);
    if (got != bytes || extra != EOF) {
        fprintf(stderr, "%s: expected %zu bytes\n", path, bytes);
        exit(1);
    }
    return buf;
}

/* A device copy of DIR/name (`bytes` bytes). */
static void* upload_file(const char* name, size_t bytes) {
    void* host = read_file(name, bytes);
    void* dev = NULL;
    CHECK(llmr_alloc(ctx, bytes, &dev));
    CHECK(llmr_upload(ctx, dev, host, bytes));
    free(host);
    return dev;
}

static void* device_buffer(size_t bytes) {
    void* dev = NULL;
    CHECK(llmr_alloc(ctx, bytes, &dev));
    return dev;
}

int main(int argc, char** argv) {
    if (argc != 6) {
        fprintf(stderr, "usage: %s DIR DIM HEADS FFN SEQ\n", argv[0]);
        return 2;
    }
    dir = argv[1];
    const uint32_t dim = (uint32_t)strtoul(argv[2], NULL, 10);
    const uint32_t heads = (uint32_t)strtoul(argv[3], NULL, 10);
    const uint32_t ffn = (uint32_t)strtoul(argv[4], NULL, 10);
    const uint32_t seq = (uint32_t)strtoul(argv[5], NULL, 10);
    if (dim != heads * 128u || dim % 32u || ffn % 32u || seq == 0) {
        fprintf(stderr, "bad shape\n");
        return 2;
    }
    const float eps = 1e-5f; /* batch_rmsnorm / batch_head_norm eps, dit.c3:1423,1447 */
    const size_t act = (size_t)seq * dim * sizeof(float);
    const size_t row_d = llmr_ggml_row_bytes(LLMR_GGML_Q8_0, dim);
    const size_t row_f = llmr_ggml_row_bytes(LLMR_GGML_Q8_0, ffn);

    CHECK(llmr_create_context(0, &ctx));

    float* hidden = upload_file("hidden.f32", act);
    void* wqkv = upload_file("wqkv.q8", 3u * dim * row_d);
    void* wo = upload_file("wo.q8", dim * row_d);
    void* w_gate = upload_file("w_gate.q8", ffn * row_d);
    void* w_up = upload_file("w_up.q8", ffn * row_d);
    void* w_down = upload_file("w_down.q8", dim * row_f);
    float* attn_norm1 = upload_file("attn_norm1.f32", dim * sizeof(float));
    float* attn_norm2 = upload_file("attn_norm2.f32", dim * sizeof(float));
    float* ffn_norm1 = upload_file("ffn_norm1.f32", dim * sizeof(float));
    float* ffn_norm2 = upload_file("ffn_norm2.f32", dim * sizeof(float));
    float* q_norm = upload_file("q_norm.f32", 128 * sizeof(float));
    float* k_norm = upload_file("k_norm.f32", 128 * sizeof(float));
    float* adaln = upload_file("adaln.f32", 4u * dim * sizeof(float)); /* scale_msa, gate_msa, scale_mlp, gate_mlp */
    float* rope_cos = upload_file("rope_cos.f32", (size_t)seq * 64 * sizeof(float));
    float* rope_sin = upload_file("rope_sin.f32", (size_t)seq * 64 * sizeof(float));

    float* buf_a = device_buffer(act);
    float* qkv = device_buffer(3 * act);
    float* slot = device_buffer(act);
    float* qh = device_buffer(act);
    float* kh = device_buffer(act);
    float* vh = device_buffer(act);
    float* attn = device_buffer(act);
    float* t = device_buffer(act);
    float* f = device_buffer((size_t)seq * ffn * sizeof(float));

    /* A: pre-attention RMSNorm, * (1 + scale_msa)                   dit.c3:1421-1432 */
    CHECK(llmr_batch_rmsnorm(ctx, hidden, dim, attn_norm1, adaln, NULL, buf_a, LLMR_GGML_F32, dim, dim, seq,
                             eps));

    /* B: Q | K | V. The reference issues three slot calls over the fused
     * [3*dim, dim] weight (row_offset 0, dim, 2*dim, dit.c3:1437-1442); the
     * same product as one call of out_dim 3*dim puts the slots side by side. */
    llmr_batch_matmul_params pc = {3u * dim, dim, seq, 0};
    CHECK(llmr_batch_matmul_pc(ctx, wqkv, LLMR_GGML_Q8_0, buf_a, LLMR_GGML_F32, qkv, &pc));
    float* fused = malloc(3 * act);
    float* one = malloc(act);
    CHECK(llmr_download(ctx, fused, qkv, 3 * act));
    int slots_equal = 1;
    for (uint32_t s = 0; s < 3; s++) {
        llmr_batch_matmul_params spc = {dim, dim, seq, s * dim};
        CHECK(llmr_batch_matmul_pc(ctx, wqkv, LLMR_GGML_Q8_0, buf_a, LLMR_GGML_F32, slot, &spc));
        CHECK(llmr_download(ctx, one, slot, act));
        for (uint32_t m = 0; m < seq && slots_equal; m++)
            if (memcmp(one + (size_t)m * dim, fused + (size_t)m * 3 * dim + (size_t)s * dim,
                       dim * sizeof(float)) != 0) {
                fprintf(stderr, "slot %u row %u differs from the fused call\n", s, m);
                slots_equal = 0;
            }
    }
    free(fused);
    free(one);

    /* C: head norm, RoPE and the head-major transpose (f32, as the
     * reference's buffers), then attention                          dit.c3:1446-1483 */
    CHECK(llmr_qkv_heads(ctx, qkv, 3u * dim, seq, heads, q_norm, k_norm, eps, rope_cos, rope_sin, qh, kh, vh,
                         LLMR_GGML_F32, seq, 0));
    llmr_flash_attention_params fa = {128u, heads, seq, 1.0f / sqrtf(128.0f)};
    CHECK(llmr_flash_attention_pc(ctx, qh, kh, vh, LLMR_GGML_F32, attn, &fa));

    /* D: O-projection; hidden += tanh(gate_msa) * rmsnorm(o-proj)    dit.c3:1488-1503 */
    pc = (llmr_batch_matmul_params){dim, dim, seq, 0};
    CHECK(llmr_batch_matmul_pc(ctx, wo, LLMR_GGML_Q8_0, attn, LLMR_GGML_F32, t, &pc));
    CHECK(llmr_gated_residual(ctx, hidden, dim, t, dim, attn_norm2, adaln + dim, LLMR_GATE_TANH, dim, seq, eps));

    /* E: FFN pre-norm, * (1 + scale_mlp)                             dit.c3:1545-1554 */
    CHECK(llmr_batch_rmsnorm(ctx, hidden, dim, ffn_norm1, adaln + 2u * dim, NULL, buf_a, LLMR_GGML_F32, dim, dim,
                             seq, eps));

    /* F: SwiGLU in-projection, down-projection                      dit.c3:1562-1596 */
    llmr_batch_matmul_params sw = {ffn, dim, seq, 0};
    CHECK(llmr_batch_matmul_swiglu_pc(ctx, w_gate, w_up, LLMR_GGML_Q8_0, buf_a, LLMR_GGML_F32, f, &sw));
    pc = (llmr_batch_matmul_params){dim, ffn, seq, 0};
    CHECK(llmr_batch_matmul_pc(ctx, w_down, LLMR_GGML_Q8_0, f, LLMR_GGML_F32, t, &pc));

    /* G: hidden += tanh(gate_mlp) * rmsnorm(down)                     dit.c3:1600-1610 */
    CHECK(llmr_gated_residual(ctx, hidden, dim, t, dim, ffn_norm2, adaln + 3u * dim, LLMR_GATE_TANH, dim, seq,
                              eps));
    CHECK(llmr_sync(ctx));

    float* out = malloc(act);
    CHECK(llmr_download(ctx, out, hidden, act));
    char path[4096];
    snprintf(path, sizeof path, "%s/out.f32", dir);
    FILE* fo = fopen(path, "wb");
    if (!fo || fwrite(out, 1, act, fo) != act) {
        fprintf(stderr, "cannot write %s\n", path);
        return 1;
    }
    fclose(fo);
    free(out);

    void* bufs[] = {hidden, wqkv,  wo,    w_gate, w_up, w_down, attn_norm1, attn_norm2, ffn_norm1,
                    ffn_norm2, q_norm, k_norm, adaln, rope_cos, rope_sin, buf_a, qkv, slot,
                    qh, kh, vh, attn, t, f};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) CHECK(llmr_free(ctx, bufs[i]));
    CHECK(llmr_destroy_context(ctx));
    printf("zimage_layer dim=%u heads=%u ffn=%u seq=%u slots_equal=%d\n", dim, heads, ffn, seq, slots_equal);
    return slots_equal ? 0 : 1;
}
