/*
 * llmr_hip.h - C-ABI of the MI355X (gfx950) backend for llm-runner's DiT
 * transformer-block hot path: GGUF block-quantized dequant-GEMM (Q8_0, Q4_K)
 * and non-causal flash attention.
 *
 * Plain C: POD arguments, device pointers as void*, sizes as uint32_t/size_t,
 * int status (0 = OK). Nothing here names a HIP or torch type, so a C3
 * `extern fn`, a ctypes stub or a C program binds it directly.
 *
 * Each entry point replaces one piece of the reference's Vulkan plumbing for
 * these ops; the citation after each declaration names the reference interface
 * it replaces (paths relative to the llm-runner tree).
 *
 * Conventions kept from the reference:
 *  - the caller owns every buffer; kernels never allocate caller-visible memory
 *    and never keep pointers across calls (Tensor ownership, lib/model/tensor.c3:8-46);
 *  - outputs are overwritten, not accumulated (llm.slang:1760-1762);
 *  - work is ordered on one in-order stream per context, so consecutive calls
 *    see each other's results without extra barriers (RenderGraph.dispatch
 *    inserts a full barrier between dispatches, lib/vulkan/graph.c3:41-61);
 *  - the host waits only at llmr_sync (RenderGraph.checkpoint/flush,
 *    lib/vulkan/graph.c3:94-107).
 * Unlike the reference (which assumes its shape preconditions), every entry
 * point validates its arguments and returns LLMR_ERR_INVALID_ARG instead of
 * launching a kernel that would read out of bounds; llmr_last_error() then
 * holds a message.
 */
#ifndef LLMR_HIP_H
#define LLMR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define LLMR_API __attribute__((visibility("default")))
#else
#define LLMR_API
#endif

/* Status codes. Any nonzero value maps to the C3 fault COMPUTE_ERROR
 * (lib/vulkan/context.c3:10). */
enum {
    LLMR_OK = 0,
    LLMR_ERR_INVALID_ARG = 1, /* shape/pointer/dtype precondition violated     */
    LLMR_ERR_UNSUPPORTED = 2, /* valid GGML type the backend does not implement */
    LLMR_ERR_HIP = 3,         /* a HIP runtime call or kernel launch failed     */
    LLMR_ERR_NO_DEVICE = 4    /* no HIP device / bad device index               */
};

/* GGML tensor type ids, same numbering as lib/gguf/types.c3:28-47. */
enum {
    LLMR_GGML_F32 = 0,
    LLMR_GGML_F16 = 1,
    LLMR_GGML_Q8_0 = 8,
    LLMR_GGML_Q4_K = 12,
    LLMR_GGML_BF16 = 30
};

/* Push-constant mirrors: identical field order and meaning to the reference's
 * 16-byte push-constant blocks. */
typedef struct llmr_batch_matmul_params {
    uint32_t out_dim;    /* N: output features written per token            */
    uint32_t in_dim;     /* K: reduction length                             */
    uint32_t seq_len;    /* M: tokens                                       */
    uint32_t row_offset; /* first weight row used (fused-weight slot select) */
} llmr_batch_matmul_params; /* BatchMatMulPC, zimage.c3l/dit.c3:172-178 */

typedef struct llmr_flash_attention_params {
    uint32_t head_dim; /* must be 128                       */
    uint32_t n_heads;
    uint32_t seq_len;
    float scale;       /* softmax scale, 1/sqrt(head_dim)   */
} llmr_flash_attention_params; /* FlashAttentionPC, zimage.c3l/dit.c3:136-142 */

typedef struct llmr_context llmr_context;

/* ---- context lifecycle ------------------------------------------------- */

/* Select HIP device `device_index` and create the context's in-order stream.
 * Replaces createContext (lib/vulkan/context.c3:73-356) for these ops. */
LLMR_API int llmr_create_context(int device_index, llmr_context** out_ctx);

/* Wait for outstanding work, destroy the stream. Replaces DeviceContext
 * teardown (lib/vulkan/context.c3:12-23). */
LLMR_API int llmr_destroy_context(llmr_context* ctx);

/* Run subsequent work on the HIP stream `hip_stream` (hipStream_t passed as
 * void*, used verbatim: NULL is the HIP null stream). Lets an embedding
 * runtime share its stream; llmr_get_stream returns the current one, so a
 * caller can save and later restore the context's own stream. No reference
 * counterpart: the reference has exactly one queue (lib/vulkan/context.c3:318-334). */
LLMR_API int llmr_set_stream(llmr_context* ctx, void* hip_stream);

/* The stream work is currently issued on (hipStream_t as void*). */
LLMR_API void* llmr_get_stream(llmr_context* ctx);

/* Message describing the last failure on the calling thread ("" if none). */
LLMR_API const char* llmr_last_error(void);

/* ---- memory ------------------------------------------------------------- */

/* Device allocation (256-byte aligned). Replaces vk::new_buffer through the
 * context allocator (lib/vulkan/context.c3:336-343, lib/model/tensor.c3:27-46). */
LLMR_API int llmr_alloc(llmr_context* ctx, size_t bytes, void** out_dev_ptr);
LLMR_API int llmr_free(llmr_context* ctx, void* dev_ptr);

/* Host->device copy of raw bytes, ordered on the context stream and complete
 * on return. Replaces upload_to_tensor / upload_weight (lib/model/tensor.c3:48-79):
 * quantized GGUF blocks are uploaded unchanged, exactly as the reference does. */
LLMR_API int llmr_upload(llmr_context* ctx, void* dst_dev, const void* src_host, size_t bytes);

/* Device->host copy, complete on return. Replaces download_tensor
 * (lib/model/tensor.c3). */
LLMR_API int llmr_download(llmr_context* ctx, void* dst_host, const void* src_dev, size_t bytes);

/* Block the host until all work issued on the context stream has finished.
 * Replaces RenderGraph.checkpoint / RenderGraph.flush (lib/vulkan/graph.c3:94-107). */
LLMR_API int llmr_sync(llmr_context* ctx);

/* ---- GGUF format helpers (host only) -------------------------------------- */

/* Bytes of one row of `n` elements of GGML type `type` (block_size/type_size,
 * lib/gguf/types.c3:50-98); 0 if the type is unknown or n is not a whole
 * number of blocks. */
LLMR_API size_t llmr_ggml_row_bytes(uint32_t type, uint32_t n);

/* ---- hot-path ops --------------------------------------------------------- */

/* Dequantize weight rows [row_offset, row_offset + n_rows) of a [*, in_dim]
 * GGUF tensor (Q8_0 or Q4_K blocks, raw GGUF layout) to f32 `out` [n_rows, in_dim].
 * Bit-exact to the reference CPU dequant: dequant_q8_0_block
 * (lib/model/tensor.c3:354-361) and dequant_q4k_block (lib/model/tensor.c3:292-335),
 * including cpu_f16_to_f32's NaN->Inf mapping (lib/model/tensor.c3:130-147). */
LLMR_API int llmr_dequant(llmr_context* ctx, const void* weight, uint32_t weight_type,
                          uint32_t n_rows, uint32_t in_dim, uint32_t row_offset, float* out);

/* Dequantize to the fp16 matrix-core operand the GEMM multiplies with, as
 * IEEE half bit patterns in `out` [n_rows, in_dim]. Q8_0: RN_fp16(fp16(d)*fp16(q)),
 * the operand of batch_matmul_q8 (dependencies/llm_text.c3l/shaders/llm.slang:1677-1705),
 * bit-exact. Q4_K: the exact value d*sc*q - dmin*mn of llm.slang:2321-2328
 * (f32 products, all exact) rounded once to fp16. */
LLMR_API int llmr_dequant_operand_f16(llmr_context* ctx, const void* weight, uint32_t weight_type,
                                      uint32_t n_rows, uint32_t in_dim, uint32_t row_offset,
                                      uint16_t* out);

/* output[m, n] = sum_k input[m, k] * W[row_offset + n, k] for m < seq_len,
 * n < out_dim, k < in_dim; output row stride is out_dim; output is overwritten.
 *   weight      raw GGUF blocks of a [>= row_offset+out_dim, in_dim] tensor,
 *               weight_type LLMR_GGML_Q8_0 (in_dim % 32 == 0) or
 *               LLMR_GGML_Q4_K (in_dim % 256 == 0); 4-byte aligned.
 *   input       [seq_len, in_dim], input_type F32, F16 or BF16; 16-byte aligned.
 *   output      f32 [seq_len, out_dim]; 16-byte aligned.
 * Replaces zimage::dispatch_batch_matmul (dependencies/zimage.c3l/dit.c3:1198-1301)
 * for Q8_0/Q4_K weights without LoRA; the caller keeps the LoRA two-hop
 * (dit.c3:1305-1364), which accumulates into `output` after this call. */
LLMR_API int llmr_batch_matmul(llmr_context* ctx, const void* weight, uint32_t weight_type,
                               const void* input, uint32_t input_type, float* output,
                               uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                               uint32_t row_offset);

/* Same op with the arguments packed as the reference's push constants
 * (g.dispatch(kernel, {weight, input, output}, &BatchMatMulPC, groups),
 * dependencies/zimage.c3l/dit.c3:1297-1300). */
LLMR_API int llmr_batch_matmul_pc(llmr_context* ctx, const void* weight, uint32_t weight_type,
                                  const void* input, uint32_t input_type, float* output,
                                  const llmr_batch_matmul_params* pc);

/* SwiGLU feed-forward in-projection, both matmuls and the activation in one op:
 *   g = input · weight_gate^T,  u = input · weight_up^T,
 *   output[s, o] = silu(g[s, o]) * u[s, o],  silu(g) = g / (1 + e^-g)
 * weight_gate and weight_up Q8_0 [out_dim, in_dim] (rows from 0), input
 * [seq_len, in_dim] of input_type F32, F16 or BF16, output f32 [seq_len,
 * out_dim], overwritten. Replaces the batch_matmul_swiglu_q8 dispatch
 * (dependencies/zimage.c3l/dit.c3:1562-1580; kernel
 * dependencies/llm_text.c3l/shaders/llm.slang:1769-1911). F32 input is
 * rounded to bf16 for the matrix cores (the reference keeps it in f32); that
 * path, and shapes the fused kernel does not take (out_dim % 4 != 0), use a
 * workspace the context allocates on first use and keeps (grow-only). */
LLMR_API int llmr_batch_matmul_swiglu(llmr_context* ctx, const void* weight_gate, const void* weight_up,
                                      uint32_t weight_type, const void* input, uint32_t input_type,
                                      float* output, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len);

/* Same op with the reference's push constants (dit.c3:1567-1579); row_offset
 * must be 0 (the reference kernel reads rows from 0). */
LLMR_API int llmr_batch_matmul_swiglu_pc(llmr_context* ctx, const void* weight_gate, const void* weight_up,
                                         uint32_t weight_type, const void* input, uint32_t input_type,
                                         float* output, const llmr_batch_matmul_params* pc);

/* Non-causal attention, no mask:
 *   out[s, h*D + d] = sum_j softmax_j(scale * <q[h,s,:], k[h,j,:]>) * v[h,j,d]
 * q, k, v [n_heads, seq_len, head_dim] of qkv_type F32, F16 or BF16 (values are
 * rounded to fp16 for the matrix cores, as the reference rounds them to fp16
 * in LDS); out f32 [seq_len, n_heads*head_dim] (reverse head transpose fused).
 * head_dim must be 128. 16-byte aligned pointers.
 * Replaces the flash_attention_v2 dispatch
 * (dependencies/zimage.c3l/dit.c3:1476-1483, dependencies/flux.c3l/flux_dit.c3:1042-1047;
 * kernel dependencies/zimage.c3l/shaders/flash_attn.slang:38-241). */
LLMR_API int llmr_flash_attention(llmr_context* ctx, const void* q, const void* k, const void* v,
                                  uint32_t qkv_type, float* out, uint32_t head_dim,
                                  uint32_t n_heads, uint32_t seq_len, float scale);

/* Same op with FlashAttentionPC packing (g.dispatch(&dk.flash_attention,
 * {Q, K, V, O}, &FlashAttentionPC, ceil(S/16), H)). */
LLMR_API int llmr_flash_attention_pc(llmr_context* ctx, const void* q, const void* k,
                                     const void* v, uint32_t qkv_type, float* out,
                                     const llmr_flash_attention_params* pc);

#ifdef __cplusplus
}
#endif

#endif /* LLMR_HIP_H */
