// llmr_internal.h - host-side launchers shared between the C-ABI layer
// (capi.hip) and the kernel translation units. Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemm_plan.h"

namespace llmr {

// Launchers return hipSuccess or the launch error; argument validation is
// done by the C-ABI layer before they are called.
hipError_t launch_dequant_f32(const void* w, uint32_t wtype, uint32_t n_rows, uint32_t in_dim,
                              uint32_t row_offset, float* out, hipStream_t st);
hipError_t launch_dequant_operand_f16(const void* w, uint32_t wtype, uint32_t n_rows,
                                      uint32_t in_dim, uint32_t row_offset, uint16_t* out,
                                      hipStream_t st);

// One GEMM (dispatch_batch_matmul). `ws` must hold
// batch_matmul_workspace_bytes(...) bytes (may be 0): f32 activations rounded
// to fp16, split-K partials of launches with few tiles and, from a few
// thousand tokens, the 16-bit weight image of the two-pass path. With a
// ws_limit the plan keeps within it where a smaller form exists (the
// one-pass kernels instead of the image, fewer splits); pass the same limit
// to both calls.
using plan::kNoWorkspaceLimit;
size_t batch_matmul_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, uint32_t M,
                                    int num_cus, size_t ws_limit = kNoWorkspaceLimit);
hipError_t launch_batch_matmul(const void* w, uint32_t wtype, const void* x, uint32_t xtype,
                               float* y, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                               uint32_t row_offset, int num_cus, void* ws, hipStream_t st,
                               size_t ws_limit = kNoWorkspaceLimit);

// Several GEMMs of one shape (N, K, weight and activation types) with a
// shared epilogue (kind kEpi* of gemm_q.hip: 0 store, 1 gated residual
// accumulate, 2 f32 | 16-bit gelu column split). Pairs of jobs run as one
// persistent launch when they fill the device; other jobs run as a plain
// GEMM into `ws` (batch_matmul_multi_workspace_bytes) plus glue passes.
struct GemmJob {
    const void* w;
    const void* x;
    float* y;
    const float* gate;
    void* y2;
    uint32_t M, row_offset;
    const float* q_norm;  // head routing (GemmEpilogue::heads): [128] or null
    const float* k_norm;
    uint32_t row0;        // sequence position of token 0
};
// Head routing of the split epilogues' first `split` = 3 n_heads 128
// columns (Q | K | V) into q, k, v [n_heads, seq, 128] of otype (16-bit):
// per job, what launch_qkv_heads computes from the f32 result.
struct GemmHeads {
    void* q;
    void* k;
    void* v;
    const float* cos;  // [seq, 64] or null
    const float* sin;
    uint32_t n_heads, seq, otype;
    float eps;
};
struct GemmEpilogue {
    uint32_t kind, ldy, ldy2, split, y2_type;
    const GemmHeads* heads;  // null, or (kind kEpiSplitGelu / kEpiSplitSwiglu) the Q | K | V routing
};
struct NextImageSet;  // the next GEMM group's weight images (below)
// prebuilt_images: the caller passes the two-pass groups' weight images
// (launch_batch_matmul_multi's `images`), so the workspace holds none.
size_t batch_matmul_multi_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K,
                                          const GemmJob* jobs, uint32_t n_jobs, const GemmEpilogue& epi,
                                          int num_cus, bool prebuilt_images = false);
// Q4_K projections of at most kGemvMaxTokens tokens, one launch for up to
// 64 jobs of one shape [N, K] with plain stores (rows ldy apart);
// hipErrorNotSupported when a job does not fit the LDS-staged kernel.
hipError_t launch_gemv_q4k_multi(uint32_t xtype, const GemmJob* jobs, uint32_t n_jobs, uint32_t N, uint32_t K,
                                 uint32_t ldy, hipStream_t st);
// images (null, or one per job): for jobs whose group runs two-pass, the
// 16-bit weight image launch_w16_image built from the job's weight, wtype,
// operand type xtype, N, K and row_offset; the group then builds none.
hipError_t launch_batch_matmul_multi(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, const GemmJob* jobs,
                                     uint32_t n_jobs, const GemmEpilogue& epi, int num_cus, void* ws,
                                     hipStream_t st, const void* const* images = nullptr,
                                     const NextImageSet* next = nullptr);

// LoRA (lora.hip): the two-hop correction appended to a base GEMM output and
// the load-time Q8_0 merge. Ranks above kMaxLoraRank are not taken (the
// reference sizes its scratch for 256).
constexpr uint32_t kMaxLoraRank = 256;
hipError_t launch_lora_correction(const float* A, const float* B, uint32_t rank, float scale, float* scratch,
                                  const void* x, uint32_t xtype, float* out, uint32_t in_dim, uint32_t out_dim,
                                  uint32_t seq_len, uint32_t b_rows, uint32_t row_offset, uint32_t weight_row_offset,
                                  hipStream_t st);
hipError_t launch_q8_lora_merge(void* base, const float* A, const float* B, uint32_t in_dim, uint32_t b_rows,
                                uint32_t dst_row_offset, uint32_t rank, float scale, hipStream_t st);

// Q4_K weights times at most kGemvMaxTokens tokens (gemv_q.hip): an
// HBM-bound weight stream, taken by launch_batch_matmul for such M.
using plan::kGemvMaxTokens;
hipError_t launch_gemv_q4k(const void* w, uint32_t xtype, const void* x, float* y, uint32_t N, uint32_t K,
                           uint32_t M, uint32_t row_offset, hipStream_t st);

// SwiGLU of two Q8_0 GEMMs (batch_matmul_swiglu_q8). `ws` must hold
// swiglu_workspace_bytes(...) bytes (may be 0).
size_t swiglu_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t out_dim, uint32_t in_dim,
                              uint32_t seq_len, int num_cus);
hipError_t launch_batch_matmul_swiglu(const void* wg, const void* wu, uint32_t wtype, const void* x,
                                      uint32_t xtype, float* y, uint32_t out_dim, uint32_t in_dim,
                                      uint32_t seq_len, int num_cus, void* ws, hipStream_t st);

// The two-pass GEMM (gemm_w16.hip): the 16-bit image of weight rows
// [row_offset, row_offset + N) (w2 non-null: the SwiGLU arrangement of gate
// w and up w2), operand type otype, into `img` (w16_image_bytes). The GEMM
// launcher itself (launch_w16_gemm) is declared in gemm_q_common.h.
using plan::w16_image_bytes;
// y = sum of the split partials part[0 .. splits) (each mn floats, mn % 4 ==
// 0), added in split order.
hipError_t launch_splitk_reduce(const float* part, float* y, uint64_t mn, uint32_t splits, hipStream_t st);
// The few-token GEMM (M <= 256, K % 64 == 0, activations f32 / f16 /
// bf16): all M tokens x 64 features per workgroup, K in `splits` non-empty
// ranges. Workspace: f32 activations rounded to fp16 (skinny_x_bytes), then,
// for splits > 1, the partials (splits * M * N floats) reduced into y.
using plan::skinny_x_bytes;
// The few-token GEMM with no K split (gemm_few.hip): M <= 256, K % 64 == 0,
// f32 / f16 / bf16 activations read in place; no workspace.
hipError_t launch_gemm_few(const void* w, uint32_t wtype, const void* x, uint32_t xtype, float* y, uint32_t N,
                           uint32_t K, uint32_t M, uint32_t row_offset, hipStream_t st);
hipError_t launch_gemm_skinny(const void* w, uint32_t wtype, const void* x, uint32_t xtype, float* y, uint32_t N,
                              uint32_t K, uint32_t M, uint32_t row_offset, uint32_t splits, void* ws,
                              hipStream_t st);
// item0 > 0: items [item0, w16_image_items(N, K, w2 != nullptr)) of the
// image, the first item0 having been built elsewhere (by the GEMM before,
// NextImageSet).
hipError_t launch_w16_image(const void* w, const void* w2, uint32_t wtype, uint32_t otype, void* img, uint32_t N,
                            uint32_t K, uint32_t row_offset, hipStream_t st, uint32_t item0 = 0);
// Work items (256-row panel x 4 stages) of a weight image (sw: the SwiGLU
// arrangement of N outputs, 128 outputs a panel).
uint32_t w16_image_items(uint32_t N, uint32_t K, bool sw = false);
// Weight images of the GEMM groups that follow a launch_batch_matmul_multi
// call (up to eight images or image parts, each its own shape, for the
// call's 16-bit input type): built in part by the two-pass GEMM's
// workgroups that are idle in its last round, the rest right after it, so
// they are complete when the next call on the stream starts. Image i: the
// plain image of rows [row_offset, + N) of w (sw 0), or the SwiGLU
// arrangement of N outputs whose gate rows are [row_offset, + N) and up
// rows [row_offset + up, + N) (sw 1; up: up[i], or N when that is 0).
constexpr uint32_t kMaxNextImages = 8;
struct NextImageSet {
    const void* w[kMaxNextImages];
    void* img[kMaxNextImages];
    uint32_t row_offset[kMaxNextImages], N[kMaxNextImages], K[kMaxNextImages], sw[kMaxNextImages];
    uint32_t up[kMaxNextImages];
    uint32_t count, wtype;
};
// Items of the images, numbered across them in order (image i's item u =
// the items of images 0..i-1 + u); the images' items from item `fused` on,
// for operand type otype.
uint32_t next_image_items(const NextImageSet& nx);
hipError_t finish_next_images(const NextImageSet& nx, uint32_t otype, uint32_t fused, hipStream_t st);
// A LoRA on a single GEMM (the reference's dispatch_batch_matmul with a
// LoRA): output columns [row_offset, row_offset + b_rows) get scale *
// b[weight_row_offset + o] . (a x).
struct LoraGemm {
    const float* a;
    const float* b;
    uint32_t rank;
    float scale;
    uint32_t b_rows, row_offset, weight_row_offset;
};
// The GEMM with its LoRA merged into the two-pass kernel's weight image
// (w + scale * b a, rounded to 16 bits once), when the GEMM runs two-pass
// and rank <= kLoraImageMaxRank: then the workspace it needs, else 0.
constexpr uint32_t kLoraImageMaxRank = 64;
// The weight image of launch_w16_image (no SwiGLU) with the LoRA merged:
// w + scale * b a on features [row_offset, row_offset + b_rows).
hipError_t launch_w16_image_lora(const void* w, uint32_t wtype, uint32_t otype, void* img, uint32_t N, uint32_t K,
                                 uint32_t row_offset, const LoraGemm& l, hipStream_t st);
size_t batch_matmul_lora_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, uint32_t M,
                                         uint32_t rank, int num_cus);
hipError_t launch_batch_matmul_lora(const void* w, uint32_t wtype, const void* x, uint32_t xtype, float* y,
                                    uint32_t N, uint32_t K, uint32_t M, uint32_t row_offset, const LoraGemm& l,
                                    int num_cus, void* ws, hipStream_t st);

// Attention (flash_attn.hip). F32 / BF16 Q, K, V are rounded to fp16 into
// `ws` first (flash_attention_workspace_bytes; 0 for F16).
size_t flash_attention_workspace_bytes(uint32_t xtype, uint32_t n_heads, uint32_t seq_len);
// The output rows: o[s * ostride + h * 128 + d] of type otype (F32, F16 or
// BF16 rounded to nearest even).
hipError_t launch_flash_attention(const void* q, const void* k, const void* v, uint32_t xtype,
                                  void* o, uint32_t otype, uint32_t ostride, uint32_t n_heads, uint32_t seq_len,
                                  float scale, void* ws, hipStream_t st);

// --- block glue (glue.hip). Strides are in elements; the C-ABI layer checks
// that every vector access is aligned (dims, strides and column offsets % 4,
// pointers 16-byte aligned) and that dims fit the kernels' register rows.

struct RowNormArgs {
    const float* x;       // [rows, x_stride] f32
    const float* w;       // [dim] RMS weight (unused by LayerNorm)
    const float* scale;   // [dim] or null: y *= 1 + scale
    const float* shift;   // [dim] or null: y += shift
    void* out;            // [rows, out_stride] of the output type
    uint32_t x_stride, out_stride, rows, dim;
    float eps;
    // rows from `split` on (a multiple of 4) take scale2 / shift2 instead
    const float* scale2 = nullptr;
    const float* shift2 = nullptr;
    uint32_t split = ~0u;
    uint32_t grid_cus = 0;  // the device's CUs (RMSNorm's persistent grid: two workgroups each)
    uint32_t grid_a = 0;    // set by the launcher: workgroups of the first side
};
constexpr uint32_t kRowNormMaxDim = 8192;

struct QkvHeadsArgs {
    const float* src;          // [rows, src_stride] f32: Q | K | V, each n_heads * 128 wide
    const float* q_norm;       // [128] or null
    const float* k_norm;       // [128] or null
    const float* rope_cos;     // [dst_seq, 64] or null
    const float* rope_sin;
    void* q;                   // [n_heads, dst_seq, 128] of the output type
    void* k;
    void* v;
    uint32_t src_stride, rows, n_heads, dst_seq, dst_row0;
    float eps;
};

struct ResidualArgs {
    float* h;               // [rows, h_stride] f32, updated in place
    const float* x;         // [rows, x_stride] f32
    const float* norm_w;    // [dim] or null: no RMSNorm of x
    const float* gate;      // [dim] or null: plain add
    uint32_t h_stride, x_stride, rows, dim;
    float eps;
    // launch_residual_norm: the updated rows' RMSNorm (weight next_w, eps
    // next_eps) * (1 + next_scale) + next_shift (either may be null) into out
    const float* next_w = nullptr;
    const float* next_scale = nullptr;
    const float* next_shift = nullptr;
    void* out = nullptr;    // [rows, out_stride] of the output type
    uint32_t out_stride = 0;
    float next_eps = 0.0f;
    uint32_t grid_cus = 0;  // the device's CUs (the persistent grid: two workgroups each)
};
// The residual update, then the updated rows' RMSNorm + modulation in the
// same pass (a.out, a.next_w non-null): bit for bit launch_residual followed
// by launch_row_norm (RMSNorm) of the residual.
hipError_t launch_residual_norm(const ResidualArgs& a, bool tanh_gate, uint32_t otype, hipStream_t st);

constexpr int kActCopy = 0, kActSilu = 1, kActGelu = 2, kActSiluMul = 3;
struct ActColsArgs {
    const float* src;   // [rows, src_stride] f32
    void* dst;          // [rows, dst_stride] of the output type
    uint32_t src_stride, src_col, src2_col, dst_stride, dst_col, rows, cols;
};

hipError_t launch_row_norm(const RowNormArgs& a, bool layernorm, uint32_t otype, hipStream_t st);
hipError_t launch_qkv_heads(const QkvHeadsArgs& a, uint32_t otype, hipStream_t st);
hipError_t launch_residual(const ResidualArgs& a, bool tanh_gate, hipStream_t st);
hipError_t launch_act_cols(const ActColsArgs& a, int act, uint32_t otype, hipStream_t st);
hipError_t launch_timestep_embed(float* out, uint32_t dim, float t, hipStream_t st);
hipError_t launch_patchify(const float* in, void* out, uint32_t otype, uint32_t C, uint32_t H, uint32_t W,
                           uint32_t ps, hipStream_t st);
hipError_t launch_unpatchify(const float* in, float* out, uint32_t C, uint32_t H, uint32_t W, uint32_t ps,
                             hipStream_t st);

// Synthetic Q4_K weights generated on the device (synth.hip): n_rows x in_dim
// values ~N(0, std^2) from a counter-based generator keyed by (seed, stream),
// quantized per 256-element superblock with the float64 min/max rule of
// llmr_amd.gguf.quantize_q4k.
hipError_t launch_synth_q4k(void* out, uint64_t n_rows, uint32_t in_dim, uint64_t seed, uint64_t stream,
                            double std, hipStream_t st);

}  // namespace llmr
