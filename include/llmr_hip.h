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

/* Bytes of the fixed scratch array of llmr_batch_matmul_noalloc. */
#define LLMR_NOALLOC_SCRATCH_BYTES (32u << 20)

/* llmr_batch_matmul that allocates nothing (no hipMalloc, hipFree or
 * allocating library call), for callers that cannot allocate: code under
 * HIP graph capture, tight serving loops, harnesses that forbid it. No
 * counterpart in the reference. Its scratch (f32 activations rounded to
 * fp16 for the persistent kernels, split-K partials of launches with few
 * tiles, the two-pass path's weight image) is a fixed
 * LLMR_NOALLOC_SCRATCH_BYTES array of device memory that each GPU holds from
 * the library's load to the end of the process. Where llmr_batch_matmul's
 * plan needs more, the call takes the form that fits: the one-pass kernels
 * instead of the weight image (the same bits), fewer K splits (the same
 * result to f32 summation order), the tiled kernel reading f32 activations
 * in place instead of their 16-bit copy (the same operands). Every call on
 * one GPU uses that GPU's one array, whose contents persist between calls.
 * Calls of one context on different streams (llmr_set_stream) are ordered
 * as its workspace is: a call on another stream than the last one waits
 * for that stream's work issued up to the switch. Calls that may overlap
 * otherwise (other contexts, other threads) race. */
LLMR_API int llmr_batch_matmul_noalloc(llmr_context* ctx, const void* weight, uint32_t weight_type,
                                       const void* input, uint32_t input_type, float* output,
                                       uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                                       uint32_t row_offset);

/* One GEMM of llmr_batch_matmul_multi: output = input · W[row_offset ..]^T as
 * llmr_batch_matmul, written through the call's epilogue. */
typedef struct llmr_matmul_job {
    const void* weight; /* raw GGUF blocks; row row_offset is output feature 0 */
    const void* input;  /* [seq_len, in_dim] of input_type, 16-byte aligned */
    float* output;      /* f32 rows, row stride ldy (GATED_RESIDUAL: read and updated) */
    const float* gate;  /* GATED_RESIDUAL: per-feature gate [out_dim], or NULL for 1 */
    void* output2;      /* SPLIT_GELU: 16-bit rows, row stride ldy2 */
    uint32_t seq_len;
    uint32_t row_offset;
} llmr_matmul_job;

enum { LLMR_EPI_STORE = 0, LLMR_EPI_GATED_RESIDUAL = 1, LLMR_EPI_SPLIT_GELU = 2, LLMR_EPI_SPLIT_SWIGLU = 3 };

/* How the f32 result r[m, n] of a job reaches memory:
 *   STORE            output[m*ldy + n] = r
 *   GATED_RESIDUAL   output[m*ldy + n] += gate[n] * r      (out_dim <= 8192)
 *   SPLIT_GELU       n <  split: output[m*ldy + n] = r
 *                    n >= split: output2[m*ldy2 + n - split] = gelu_tanh(r)
 *                    rounded to output2_type (split % 8 == 0)
 *   SPLIT_SWIGLU     out_dim = split + 2 f: weight rows [split, split + f)
 *                    are a SwiGLU gate, [split + f, split + 2 f) its up:
 *                    n < split: output[m*ldy + n] = r;
 *                    o < f: output2[m*ldy2 + o] = silu(r[split + o]) *
 *                    r[split + f + o] rounded to output2_type
 *                    (split % 256 == 0, f % 8 == 0)
 * ldy 0 means out_dim (SPLIT_*: split); ldy2 0 means out_dim - split
 * (SPLIT_SWIGLU: f). Strides are multiples of 4; out_dim % 4 == 0 unless the
 * epilogue is a STORE with ldy == out_dim. */
typedef struct llmr_matmul_epilogue {
    uint32_t kind;
    uint32_t ldy;
    uint32_t split;
    uint32_t ldy2;
    uint32_t output2_type; /* LLMR_GGML_BF16 or LLMR_GGML_F16 */
} llmr_matmul_epilogue;

/* n_jobs GEMMs of one shape and type (out_dim, in_dim, weight_type,
 * input_type) with a shared epilogue (NULL: STORE, ldy = out_dim). Equivalent
 * to n_jobs llmr_batch_matmul calls each followed by its epilogue; the jobs'
 * outputs must not overlap. Replaces the reference's per-stream and per-slot
 * dispatch_batch_matmul calls and the glue dispatches that follow them:
 *   - the image and text stream projections of a Flux double block
 *     (dependencies/flux.c3l/flux_dit.c3:786-804, 875-887, 917-964), run as
 *     one launch: pairs of jobs share the device as one grid of tiles;
 *   - gated_residual_linear after a projection (flux_dit.c3:891-898, 1064-1068);
 *   - the single block's linear1 slots plus silu/gelu and concat_rows_copy
 *     (flux_dit.c3:1005-1018, 1049-1058): Q | K | V to `output`, the
 *     activated MLP half straight into linear2's input (SPLIT_SWIGLU: the
 *     reference's Flux.2 block, silu(gate) * up of linear1's last 2 f rows,
 *     flux_dit.c3:1013-1018, 1049-1055; SPLIT_GELU: the Flux.1 form);
 *   - a double block's MLP in-projection and its SwiGLU (SPLIT_SWIGLU with
 *     split 0: flux_dit.c3:917-931, 945-955), both streams in one launch;
 *   - the modulation projections of one step (the reference makes three
 *     shared ones, flux_dit.c3:1131-1140; a Flux.1-dev model has one per block):
 *     Q4_K jobs of at most 4 tokens with LLMR_EPI_STORE run as one launch
 *     for the whole group.
 * A job pair that cannot run as one persistent launch (f32 input, too few
 * tiles, ...) runs job by job through a context workspace (grow-only, like
 * the SwiGLU's). No reference counterpart as a single call. */
LLMR_API int llmr_batch_matmul_multi(llmr_context* ctx, uint32_t weight_type, uint32_t input_type,
                                     uint32_t out_dim, uint32_t in_dim, const llmr_matmul_job* jobs,
                                     uint32_t n_jobs, const llmr_matmul_epilogue* epilogue);

/* Weight images built ahead of the GEMM. From a few thousand tokens a GEMM
 * runs in two passes: its weight rows are first dequantized into a 16-bit
 * image (laid out as the GEMM's LDS tiles), which the matrix-core pass then
 * streams. A caller that knows its next GEMM group (a whole denoising step)
 * can have each call build the next group's images, or the next two groups'
 * where its idle workgroups have room: the current GEMM's workgroups that
 * have no tile in its last round build what fits, the rest runs right after
 * it. No reference counterpart (the reference
 * dequantizes inside every matmul dispatch, llm.slang:1677-1705, 2321-2328);
 * the results are bit-identical to llmr_batch_matmul_multi.
 *
 * llmr_weight_image_bytes: bytes of the image of out_dim rows of in_dim
 * (0 when in_dim % 64 != 0).
 * llmr_build_weight_image: rows [row_offset, row_offset + out_dim) of a
 * Q8_0 / Q4_K weight into `image` (256-byte aligned, image_bytes >= the size
 * above), as operands for input_type F16 or BF16, on the context's current
 * stream. */
LLMR_API size_t llmr_weight_image_bytes(uint32_t out_dim, uint32_t in_dim);
/* Bytes of the SwiGLU-arranged image of n_out outputs (gate and up rows
 * interleaved per 128 outputs; 0 when in_dim % 64 != 0). */
LLMR_API size_t llmr_swiglu_weight_image_bytes(uint32_t n_out, uint32_t in_dim);
LLMR_API int llmr_build_weight_image(llmr_context* ctx, const void* weight, uint32_t weight_type,
                                     uint32_t input_type, uint32_t out_dim, uint32_t in_dim, uint32_t row_offset,
                                     void* image, size_t image_bytes);

/* One weight image a call builds for a later call, of a weight with in_dim
 * columns. swiglu 0: rows [row_offset, row_offset + out_dim) (sized by
 * llmr_weight_image_bytes). swiglu 1: the SwiGLU arrangement of out_dim
 * outputs, gate rows [row_offset, row_offset + out_dim) and up rows
 * [row_offset + u, row_offset + u + out_dim) with u = up_offset, or out_dim
 * when up_offset is 0 (sized by llmr_swiglu_weight_image_bytes): what a
 * SPLIT_SWIGLU job reads after the plain image of its first `split` rows,
 * at llmr_weight_image_bytes(split, in_dim) into its image. A part of an
 * image is an image too: the rows [256 p0, 256 p1) of a plain image (row
 * offset + 256 p0) start p0 panels into it, the outputs [128 p0, 128 p1)
 * of a SwiGLU image of f outputs (row offset + 128 p0, up_offset f) p0
 * panels in, a panel being llmr_weight_image_bytes(256, in_dim) bytes. */
typedef struct llmr_next_weight_image {
    const void* weight;
    uint32_t out_dim;
    uint32_t in_dim;     /* % 64 == 0 */
    uint32_t row_offset;
    uint32_t swiglu;
    uint32_t up_offset;  /* swiglu 1 only; 0: out_dim */
    void* image;         /* 256-byte aligned */
    size_t image_bytes;
} llmr_next_weight_image;

/* The weight images of the GEMM groups a caller issues next: `count` (1 to
 * 8) images or image parts of weights of weight_type, for the same
 * input_type as the call that builds them. */
typedef struct llmr_next_weight_images {
    uint32_t weight_type;
    uint32_t count;
    llmr_next_weight_image image[8];
} llmr_next_weight_images;

/* llmr_batch_matmul_multi, plus:
 *   images (NULL, or one per job): images[i] = the image of job i's weight,
 *     built by llmr_build_weight_image or by the `next` of an earlier call
 *     with the job's weight, weight_type, input_type, out_dim, in_dim and
 *     row_offset (the weight unchanged since; the call cannot check the
 *     contents). SPLIT_SWIGLU: the image of rows [row_offset, + split) (none
 *     when split == 0), then at llmr_weight_image_bytes(split, in_dim) the
 *     SwiGLU image of the job's f outputs (a `next` entry with swiglu 1,
 *     out_dim f, row_offset + split). Job groups that run two-pass use them
 *     instead of building their own; other groups ignore them.
 *   next (NULL or images of later groups): all built before the call
 *     returns its work to the stream, as many items as fit by this call's
 *     idle workgroups (the workgroups without a tile in the GEMM's last
 *     round), the rest by an image launch right after the GEMM. None may be
 *     an image this call reads.
 * Either needs input_type F16 or BF16. */
LLMR_API int llmr_batch_matmul_multi_images(llmr_context* ctx, uint32_t weight_type, uint32_t input_type,
                                            uint32_t out_dim, uint32_t in_dim, const llmr_matmul_job* jobs,
                                            uint32_t n_jobs, const llmr_matmul_epilogue* epilogue,
                                            const void* const* images, const llmr_next_weight_images* next);

/* Head routing of a QKV projection's result, per job (NULL: no norms, row0 0). */
typedef struct llmr_qkv_heads_job {
    const float* q_norm; /* [128] or NULL (16-byte aligned) */
    const float* k_norm; /* [128] or NULL */
    uint32_t row0;       /* sequence position of the job's token 0 */
} llmr_qkv_heads_job;

/* The Q | K | V columns of a QKV projection routed to the attention's
 * head-major inputs, as llmr_qkv_heads does from the f32 result. */
typedef struct llmr_qkv_heads_out {
    void* q;                        /* [n_heads, seq_len, 128] of out_type each, 16-byte aligned */
    void* k;
    void* v;
    uint32_t out_type;              /* LLMR_GGML_F16 or LLMR_GGML_BF16 */
    uint32_t n_heads;
    uint32_t seq_len;
    float eps;
    const float* rope_cos;          /* [seq_len, 64] f32, or both NULL */
    const float* rope_sin;
    const llmr_qkv_heads_job* jobs; /* n_jobs entries, or NULL */
} llmr_qkv_heads_out;

/* llmr_batch_matmul_multi_images, with the result's first 3 * n_heads * 128
 * columns (Q | K | V; the whole result for a STORE epilogue, [0, split) for
 * SPLIT_GELU and SPLIT_SWIGLU, GATED_RESIDUAL not taken) written through
 * `heads` instead of to the jobs' `output` (which may then be NULL): for
 * job i, llmr_qkv_heads(result rows, n_heads, jobs[i].q_norm, jobs[i].k_norm,
 * eps, rope tables, q, k, v, out_type, seq_len, jobs[i].row0), bit for bit
 * (the row's sum of squares in the same order). row0 + seq_len of each job
 * <= heads->seq_len. The persistent GEMM launches do it in their epilogue,
 * so the f32 Q | K | V never reaches memory; other job groups run the GEMM
 * into the context workspace and then llmr_qkv_heads. Replaces a QKV
 * dispatch_batch_matmul followed by batch_head_norm x2 + transpose_heads x3
 * + mrope x2 (dependencies/zimage.c3l/dit.c3:1434-1473,
 * dependencies/flux.c3l/flux_dit.c3:786-863, 1005-1040). */
LLMR_API int llmr_batch_matmul_multi_qkv(llmr_context* ctx, uint32_t weight_type, uint32_t input_type,
                                         uint32_t out_dim, uint32_t in_dim, const llmr_matmul_job* jobs,
                                         uint32_t n_jobs, const llmr_matmul_epilogue* epilogue,
                                         const llmr_qkv_heads_out* heads, const void* const* images,
                                         const llmr_next_weight_images* next);

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

/* ---- GGUF checkpoints (host side) -------------------------------------------- */

/* An open GGUF file: gguf_parse (lib/gguf/parser.c3:164-208) over a
 * read-only memory map. Versions 2 and 3; tensor data aligned to 32 bytes
 * after the tensor infos (the reference's hard-coded alignment,
 * lib/gguf/types.c3:8). Every read is bounds-checked: a truncated or corrupt
 * file gives LLMR_ERR_INVALID_ARG. Strings and data pointers returned below
 * point into the handle and stay valid until llmr_gguf_close. */
typedef struct llmr_gguf llmr_gguf;

/* GGUFTensorInfo (parser.c3:135-160): ne[] fastest-varying first (a row-major
 * [out, in] weight has ne = {in, out}), unused dims 1; offset relative to the
 * data section; data_size = ceil(elements / block_size) * type_size
 * (GGMLType tables, types.c3:50-98; 0 for an unknown type); data = the
 * tensor's bytes in the mapping. */
typedef struct llmr_gguf_tensor_info {
    const char* name;
    uint32_t type;
    uint32_t n_dims;
    uint64_t ne[4];
    uint64_t offset;
    uint64_t data_size;
    const void* data;
} llmr_gguf_tensor_info;

/* GGUFMetaKV (parser.c3:94-133): type is the GGUFType (0 UINT8 ... 7 BOOL,
 * 8 STRING, 9 ARRAY, 10 UINT64, 11 INT64, 12 FLOAT64); data points at the
 * value (a scalar's bytes; a string's bytes, data_len long, not
 * NUL-terminated; an array's elements, array_len of array_type, strings
 * each prefixed by their u64 length). */
typedef struct llmr_gguf_kv_info {
    const char* key;
    uint32_t type;
    uint32_t array_type;
    uint64_t array_len;
    const void* data;
    uint64_t data_len;
} llmr_gguf_kv_info;

LLMR_API int llmr_gguf_open(const char* path, llmr_gguf** out);
LLMR_API int llmr_gguf_close(llmr_gguf* gguf);
LLMR_API int llmr_gguf_info(const llmr_gguf* gguf, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv);
LLMR_API int llmr_gguf_tensor(const llmr_gguf* gguf, uint64_t index, llmr_gguf_tensor_info* out);
/* GGUFFile.find_tensor (parser-side lookup used by load_dit_tensor, flux_dit.c3:191-207) */
LLMR_API int llmr_gguf_find_tensor(const llmr_gguf* gguf, const char* name, uint64_t* index);
LLMR_API int llmr_gguf_kv(const llmr_gguf* gguf, uint64_t index, llmr_gguf_kv_info* out);
LLMR_API int llmr_gguf_find_kv(const llmr_gguf* gguf, const char* key, uint64_t* index);

/* upload_weight (lib/model/tensor.c3:48-66): the tensor's bytes, unchanged
 * (quantized blocks in their GGUF layout), into a device buffer of at least
 * data_size bytes; complete on return. llmr_gguf_load_tensor allocates that
 * buffer (llmr_alloc; release it with llmr_free) as upload_weight does.
 * LLMR_ERR_UNSUPPORTED for a type of unknown size. */
LLMR_API int llmr_gguf_upload_tensor(llmr_context* ctx, const llmr_gguf* gguf, uint64_t index, void* dst_dev,
                                     size_t dst_bytes);
LLMR_API int llmr_gguf_load_tensor(llmr_context* ctx, const llmr_gguf* gguf, uint64_t index, void** out_dev_ptr);

/* ---- LoRA ------------------------------------------------------------------ */

/* A LoRA adapter of one linear (LoraTensor, lib/model/lora.c3:22-28): a
 * [rank, in_dim] and b [out_rows, rank], f32 device pointers; the correction
 * is scale * (b . a). */
typedef struct llmr_lora {
    const float* a;
    const float* b;
    uint32_t rank;
    float scale;
} llmr_lora;

/* The two-hop LoRA correction appended to a base llmr_batch_matmul output
 * (dispatch_lora_correction, dependencies/zimage.c3l/dit.c3:1319-1364):
 *   hop 1: scratch[s, r] = sum_k a[r, k] * input[s, k]
 *          (batch_matmul_simple, llm.slang:1146-1180; the sum in the order of
 *          a 256-thread workgroup: strided partials, then the tree)
 *   hop 2: output[s * out_dim + row_offset + o] += lora.scale *
 *          sum_r b[weight_row_offset + o, r] * scratch[s, r]   for o < b_rows
 *          (batch_matmul_add_scaled, llm.slang:1262-1294; the sum in r order)
 * input [seq_len, in_dim] of input_type F32, F16 or BF16 (widened exactly);
 * output f32 with row stride out_dim, accumulated. b_rows 0 means out_dim.
 * scratch: seq_len * rank floats on the device, caller-owned (the
 * reference's lora_scratch). Bit-identical to the CPU restatement. lora
 * NULL or rank 0 or rank > 256: nothing is done and
 * LLMR_OK is returned, as the reference skips those. The dot products are
 * fused multiply-adds (the reference leaves contraction to its shader
 * compiler). */
LLMR_API int llmr_lora_correction(llmr_context* ctx, const llmr_lora* lora, float* scratch, const void* input,
                                  uint32_t input_type, float* output, uint32_t in_dim, uint32_t out_dim,
                                  uint32_t seq_len, uint32_t b_rows, uint32_t row_offset,
                                  uint32_t weight_row_offset);

/* llmr_batch_matmul with its LoRA, the reference's dispatch_batch_matmul
 * with a LoRA (dit.c3:1198-1213: lora, lora_scratch, lora_b_rows,
 * lora_row_offset, lora_weight_row_offset). lora NULL: the plain GEMM. A GEMM
 * on the two-pass kernel (seq_len >= 2048, at least half the CUs' worth of
 * 256 x 256 tiles) with rank <= 64 merges the adapter into its 16-bit weight
 * image: W' = RN16(W16 + scale * b a) on output features [lora_row_offset,
 * lora_row_offset + b_rows), one more 16-bit rounding of those weights
 * (within the GEMM's tolerance of the reference; the other features are
 * bit-identical to llmr_batch_matmul), lora_scratch unused. Every other
 * call is llmr_batch_matmul followed by llmr_lora_correction. */
LLMR_API int llmr_batch_matmul_lora(llmr_context* ctx, const void* weight, uint32_t weight_type,
                                    const void* input, uint32_t input_type, float* output, uint32_t out_dim,
                                    uint32_t in_dim, uint32_t seq_len, uint32_t row_offset, const llmr_lora* lora,
                                    float* lora_scratch, uint32_t lora_b_rows, uint32_t lora_row_offset,
                                    uint32_t lora_weight_row_offset);

/* Folds scale * (b . a) into rows [dst_row_offset, dst_row_offset + b_rows)
 * of a Q8_0 weight [*, in_dim] in place and requantizes each 32-element
 * block (q8_lora_merge, dependencies/llm_text.c3l/shaders/llm.slang:1337-1420;
 * host merge_one_site, dependencies/flux.c3l/lora_merge.c3:36-73):
 *   u = d * q + scale * sum_r b[j, r] * a[r, k]   (fused sum in r order)
 *   d' = max(absmax(u over the block) / 127, 1e-8); q' = clamp(round(u / d'),
 *   -127, 127) with halves away from zero (trunc(u/d' +- 0.5) in f32);
 *   d' stored as f16, round to nearest even.
 * b is [b_rows, rank]. in_dim % 256 == 0 and 1 <= rank <= 256
 * (LLMR_ERR_UNSUPPORTED otherwise: the reference skips such merges and keeps
 * the runtime correction). Bit-identical to the CPU restatement. */
LLMR_API int llmr_q8_lora_merge(llmr_context* ctx, void* weight, const float* a, const float* b, uint32_t in_dim,
                                uint32_t b_rows, uint32_t dst_row_offset, uint32_t rank, float scale);

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

/* llmr_flash_attention with the output rows written straight into the next
 * projection's input: out[s * out_stride + h * head_dim + d] of out_type
 * (F32, or F16 / BF16 rounded to nearest even from the f32 result, the
 * values llmr_activation's ACT_COPY gives), out_stride % 8 == 0 and >=
 * n_heads * head_dim, out 16-byte aligned. Replaces the attention dispatch
 * plus the copy that follows it in a block (dit.c3:1476-1487,
 * flux_dit.c3:865-872, 1042-1047). No reference counterpart as one call. */
LLMR_API int llmr_flash_attention_rows(llmr_context* ctx, const void* q, const void* k, const void* v,
                                       uint32_t qkv_type, void* out, uint32_t out_type, uint32_t out_stride,
                                       uint32_t head_dim, uint32_t n_heads, uint32_t seq_len, float scale);

/* Same op with FlashAttentionPC packing (g.dispatch(&dk.flash_attention,
 * {Q, K, V, O}, &FlashAttentionPC, ceil(S/16), H)). */
LLMR_API int llmr_flash_attention_pc(llmr_context* ctx, const void* q, const void* k,
                                     const void* v, uint32_t qkv_type, float* out,
                                     const llmr_flash_attention_params* pc);

/* ---------------------------------------------------------------------------
 * Block glue: the row reductions and elementwise ops the DiT blocks run
 * between the GEMMs and attention. Each replaces a chain of the reference's
 * dispatches over one tensor with one pass, and writes its result directly in
 * the type the next GEMM or attention call reads (out_type F32, F16 or BF16),
 * so a block never round-trips f32 activations through memory just to convert
 * them. All math is f32 in the reference's operation order.
 * Shared preconditions: dims, row strides and column offsets are in elements
 * and multiples of 4 (8-byte / 16-byte vector accesses); pointers 16-byte
 * aligned; row widths (dim) at most 8192. Strides let a call address a row
 * range or column slice of a larger buffer (e.g. the image rows of a joint
 * text+image sequence) without a copy.
 * ------------------------------------------------------------------------- */

enum { LLMR_ACT_COPY = 0, LLMR_ACT_SILU = 1, LLMR_ACT_GELU_TANH = 2, LLMR_ACT_SILU_MUL = 3 };
enum { LLMR_GATE_NONE = 0, LLMR_GATE_LINEAR = 1, LLMR_GATE_TANH = 2 };

/* out[r, d] = x[r, d] * (1 / sqrt(sum_d x[r, d]^2 / dim + eps)) * weight[d],
 * then *= 1 + mod_scale[d] and += mod_shift[d] where those are non-null.
 * x f32 [n_rows, x_stride], out [n_rows, out_stride] of out_type.
 * Replaces batch_rmsnorm followed by scale_modulate
 * (dependencies/zimage.c3l/dit.c3:1424-1432, 1546-1554; kernels
 * dependencies/zimage.c3l/shaders/zimage.slang:449-500, 356-373). */
LLMR_API int llmr_batch_rmsnorm(llmr_context* ctx, const float* x, uint32_t x_stride, const float* weight,
                                const float* mod_scale, const float* mod_shift, void* out, uint32_t out_type,
                                uint32_t out_stride, uint32_t dim, uint32_t n_rows, float eps);

/* out[r, d] = (x[r, d] - mean_r) * (1 / sqrt(var_r + eps)) (no affine;
 * two-pass mean and variance), then *= 1 + mod_scale[d] and += mod_shift[d]
 * where non-null. Replaces batch_layernorm followed by adaln_modulate
 * (dependencies/flux.c3l/flux_dit.c3:767-770, 992-995, 1186-1191; kernels
 * zimage.slang:502-561, 98-117). */
LLMR_API int llmr_batch_layernorm(llmr_context* ctx, const float* x, uint32_t x_stride, const float* mod_scale,
                                  const float* mod_shift, void* out, uint32_t out_type, uint32_t out_stride,
                                  uint32_t dim, uint32_t n_rows, float eps);

/* llmr_batch_layernorm over rows that belong to two streams with their own
 * modulation: rows [0, split_row) take mod_scale / mod_shift, rows
 * [split_row, n_rows) mod_scale2 / mod_shift2 (each pair may hold nulls);
 * split_row % 4 == 0. One launch for the Flux double block's text and image
 * streams, which the reference normalizes by two batch_layernorm +
 * adaln_modulate dispatches each (dependencies/flux.c3l/flux_dit.c3:761-779,
 * 903-909, 939-945); the rows equal those two calls' bit for bit. */
LLMR_API int llmr_batch_layernorm_split(llmr_context* ctx, const float* x, uint32_t x_stride,
                                        const float* mod_scale, const float* mod_shift, uint32_t split_row,
                                        const float* mod_scale2, const float* mod_shift2, void* out,
                                        uint32_t out_type, uint32_t out_stride, uint32_t dim, uint32_t n_rows,
                                        float eps);

/* Per-head RMSNorm + rotary embedding + head-major transpose of a QKV GEMM
 * output. qkv f32 [n_rows, qkv_stride] holds Q | K | V, each n_heads*128
 * wide, starting at column 0. For row r (sequence position t = row0 + r),
 * head h, pair j < 64:
 *   x = qkv[r, slot*n_heads*128 + h*128 + 2j .. 2j+1]
 *   Q, K: x *= (1 / sqrt(sum_head x^2 / 128 + eps)) * norm[2j .. 2j+1]   (norm non-null)
 *   Q, K: (x0, x1) -> (x0*c - x1*s, x0*s + x1*c), c/s = rope_cos/sin[t, j]
 *         (tables f32 [seq_len, 64], both null for no rotation)
 *   out_slot[h, t, 2j .. 2j+1] = x    (q, k, v [n_heads, seq_len, 128] of out_type)
 * row0 + n_rows <= seq_len; the tables must hold seq_len rows. Replaces
 * batch_head_norm x2 + transpose_heads x3 + mrope x2
 * (dependencies/zimage.c3l/dit.c3:1448-1473, dependencies/flux.c3l/flux_dit.c3:
 * 814-863, 1022-1040; kernels zimage.slang:563-667,
 * dependencies/zimage.c3l/shaders/mrope.slang:33-54). Two calls with
 * different norms and row0 fill the text and image rows of a joint sequence. */
LLMR_API int llmr_qkv_heads(llmr_context* ctx, const float* qkv, uint32_t qkv_stride, uint32_t n_rows,
                            uint32_t n_heads, const float* q_norm, const float* k_norm, float eps,
                            const float* rope_cos, const float* rope_sin, void* q, void* k, void* v,
                            uint32_t out_type, uint32_t seq_len, uint32_t row0);

/* residual[r, d] += g * y with y = input[r, d], RMS-normalised with
 * norm_weight first when that is non-null (eps as batch_rmsnorm), and
 *   LLMR_GATE_NONE:   g * y = y                          (residual_add)
 *   LLMR_GATE_LINEAR: g * y = gate[d] * y                (gated_residual_linear)
 *   LLMR_GATE_TANH:   clamp(tanh(gate[d]) * y, +-1e10)   (gated_residual, scale 1)
 * residual f32 [n_rows, residual_stride] updated in place, input f32.
 * Replaces the post-norm + gated residual pairs of the Z-Image block
 * (dependencies/zimage.c3l/dit.c3:1495-1503, 1602-1610) and Flux's
 * gated_residual_linear (dependencies/flux.c3l/flux_dit.c3:891-898, 1067-1068;
 * kernels zimage.slang:382-424, lib/shaders/diffusion.slang:1713-1716). */
LLMR_API int llmr_gated_residual(llmr_context* ctx, float* residual, uint32_t residual_stride, const float* input,
                                 uint32_t input_stride, const float* norm_weight, const float* gate,
                                 uint32_t gate_mode, uint32_t dim, uint32_t n_rows, float eps);

/* llmr_gated_residual, then in the same pass over the rows
 * llmr_batch_rmsnorm of the updated residual with next_weight (non-null),
 * next_scale and next_shift (each may be null) and next_eps into out (of
 * out_type): the Z-Image block's attention post-norm + gated residual and
 * its FFN pre-norm (dependencies/zimage.c3l/dit.c3:1495-1503 then
 * 1545-1554), bit for bit those two calls, reading and writing the residual
 * rows once. dim <= 4096. No reference counterpart as a single dispatch. */
LLMR_API int llmr_gated_residual_rmsnorm(llmr_context* ctx, float* residual, uint32_t residual_stride,
                                         const float* input, uint32_t input_stride, const float* norm_weight,
                                         const float* gate, uint32_t gate_mode, const float* next_weight,
                                         const float* next_scale, const float* next_shift, void* out,
                                         uint32_t out_type, uint32_t out_stride, uint32_t dim, uint32_t n_rows,
                                         float eps, float next_eps);

/* dst[r, dst_col + c] = f(src[r, src_col + c]) for c < n_cols with
 *   LLMR_ACT_COPY      x                         (a cast / column copy)
 *   LLMR_ACT_SILU      x / (1 + exp(-x))
 *   LLMR_ACT_GELU_TANH 0.5*x*(1 + tanh(0.7978845608*(x + 0.044715*x^3)))
 *   LLMR_ACT_SILU_MUL  silu(x) * src[r, src2_col + c]
 * src f32 [n_rows, src_stride]; dst [n_rows, dst_stride] of dst_type.
 * Replaces silu + elemwise_mul (dependencies/flux.c3l/flux_dit.c3:929-931,
 * 1051-1053; kernels lib/shaders/diffusion.slang:1082-1086, 1733-1736), gelu
 * (diffusion.slang:1092-1107) and the single-stream concat_rows_copy
 * (flux_dit.c3:625-660, 1057): the
 * attention output and the activated MLP half are written into the column
 * ranges [0, dim) and [dim, dim + mlp) of linear2's input. */
LLMR_API int llmr_activation(llmr_context* ctx, const float* src, uint32_t src_stride, uint32_t src_col,
                             uint32_t src2_col, void* dst, uint32_t dst_type, uint32_t dst_stride, uint32_t dst_col,
                             uint32_t n_rows, uint32_t n_cols, uint32_t act);

/* out[i] = cos(t * f_i) for i < dim/2 and sin(t * f_(i - dim/2)) above, with
 * f_j = exp(-ln(10000) * j / (dim/2)); dim even. Replaces dit_timestep_embed
 * (dependencies/flux.c3l/flux_dit.c3:1121-1123; kernel zimage.slang:284-307). */
LLMR_API int llmr_timestep_embed(llmr_context* ctx, float* out, uint32_t dim, float timestep);

/* latent f32 [channels, height, width] -> out [(height/p)*(width/p),
 * channels*p*p] of out_type, element (py*p + px)*channels + c of each patch.
 * Replaces patchify (dependencies/flux.c3l/flux_dit.c3:1096-1100; kernel
 * zimage.slang:11-51). */
LLMR_API int llmr_patchify(llmr_context* ctx, const float* latent, void* out, uint32_t out_type,
                           uint32_t channels, uint32_t height, uint32_t width, uint32_t patch_size);

/* The inverse permutation, f32 (unpatchify, flux_dit.c3:1196-1202; kernel
 * zimage.slang:56-93). */
LLMR_API int llmr_unpatchify(llmr_context* ctx, const float* patches, float* out, uint32_t channels,
                             uint32_t height, uint32_t width, uint32_t patch_size);

/* Synthetic Q4_K weights generated on the device: out receives
 * n_rows * in_dim/256 blocks (144 B each) of values ~N(0, std^2) drawn from
 * the counter-based stream (seed, stream) and quantized per superblock.
 * Byte-identical to the host-side generator + quantizer of the Python
 * package (llmr_amd.synth.normal, llmr_amd.gguf.quantize_q4k). Test and
 * benchmark setup only; the reference loads real GGUF weights instead
 * (lib/model/tensor.c3:48-66). in_dim % 256 == 0. */
LLMR_API int llmr_synth_q4k(llmr_context* ctx, void* out, uint64_t n_rows, uint32_t in_dim, uint64_t seed,
                            uint64_t stream, double std);

#ifdef __cplusplus
}
#endif

#endif /* LLMR_HIP_H */
