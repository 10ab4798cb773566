// glue.hip - the DiT block's row-reduction and elementwise ops around the
// GEMMs and flash attention (dependencies/zimage.c3l/shaders/zimage.slang,
// mrope.slang, lib/shaders/diffusion.slang), each a single pass over its
// data. Where the reference issues a chain of dispatches over one tensor, the
// chain is one kernel here:
//   row_norm       batch_rmsnorm | batch_layernorm, then scale_modulate |
//                  adaln_modulate, written straight in the next GEMM's
//                  activation type (f32 / f16 / bf16)
//   qkv_heads      batch_head_norm + transpose_heads + mrope on the Q/K/V
//                  slots of one QKV (or linear1) GEMM output
//   residual       batch_rmsnorm (optional) + gated_residual |
//                  gated_residual_linear | residual_add into the f32 stream
//   act_cols       silu / gelu / silu*mul / copy over a column range, written
//                  into a column range of another tensor (the single-stream
//                  concat) in the next GEMM's activation type
// plus the timestep embedding and (un)patchify. Arithmetic is f32 in the
// reference's operation order; floating-point contraction is off in this file
// so products and sums round where the reference's source writes them.
#include <hip/hip_runtime.h>

#include "llmr_device.h"
#include "llmr_internal.h"

#pragma clang fp contract(off)

namespace llmr {
namespace {

// Workgroups of a persistent row-group kernel: two per CU (cus 0: one per
// group of four rows). Measured on the Z-Image residual kernels (4352 rows,
// 1088 groups): 512 workgroups of two or three groups beat 363 of three
// (more rows in flight) and 1088 of one (the vectors staged 1088 times).
inline uint32_t persistent_grid(uint32_t rows, uint32_t cus) {
    const uint32_t quads = (rows + 3u) / 4u;
    return cus ? min(quads, 2u * cus) : quads;
}

// --- output conversion -------------------------------------------------------

template <uint32_t OT>
__device__ __forceinline__ void store4(void* base, size_t idx, f32x4 v) {
    if constexpr (OT == kGgmlF32) {
        *(f32x4*)((float*)base + idx) = v;
    } else if constexpr (OT == kGgmlF16) {
        *(u32x2*)((uint16_t*)base + idx) = u32x2{pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w)};
    } else {
        typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
        bf16x4_t b;
        b.x = (__bf16)v.x;  // round to nearest even
        b.y = (__bf16)v.y;
        b.z = (__bf16)v.z;
        b.w = (__bf16)v.w;
        *(bf16x4_t*)((uint16_t*)base + idx) = b;
    }
}

template <uint32_t OT>
__device__ __forceinline__ void store2(void* base, size_t idx, float a, float b) {
    if constexpr (OT == kGgmlF32) {
        *(f32x2*)((float*)base + idx) = f32x2{a, b};
    } else if constexpr (OT == kGgmlF16) {
        *(uint32_t*)((uint16_t*)base + idx) = pack_f16x2(a, b);
    } else {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        bf16x2_t r;
        r.x = (__bf16)a;
        r.y = (__bf16)b;
        *(bf16x2_t*)((uint16_t*)base + idx) = r;
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ f32x4 ld4(const float* p) { return *(const f32x4*)p; }

// --- row_norm ----------------------------------------------------------------
// One wave per row, the row held in registers (NV float4 per lane, so
// dim <= 256 * NV). RMS (zimage.slang:465-500):
//   y = x * (1 / sqrt(sum(x^2) / dim + eps)) * w[d]
// LayerNorm without affine, two passes (zimage.slang:517-561):
//   y = (x - mean) * (1 / sqrt(sum((x - mean)^2) / dim + eps))
// then, when given, y = y * (1 + scale[d]) (scale_modulate, zimage.slang:368-
// 373) and y = y + shift[d] (adaln_modulate, zimage.slang:111-117).

template <bool LN, uint32_t OT, int NV>
__global__ void __launch_bounds__(256) row_norm_kernel(RowNormArgs a) {
    // The vectors of one side of the split (1 + scale, shift; RMSNorm: its
    // weight too), staged once per workgroup (element 4k .. 4k+3 at k); the
    // workgroups of a side walk its groups of four rows. LayerNorm launches
    // one workgroup per group (with two staged vectors they fit one round,
    // five per CU, at the Flux shapes), RMSNorm a persistent grid of two per
    // CU (three vectors of d = 3840: one group each ran in two rounds and
    // staged the vectors per group).
    constexpr int kW = LN ? -1 : 0, kS = LN ? 0 : 1, kH = LN ? 1 : 2;
    __shared__ f32x4 vec_lds[LN ? 2 : 3][NV * 64];
    const uint32_t lane = threadIdx.x & 63u;
    // side one: groups [0, qa) (all of them without a split; split % 4 == 0)
    const uint32_t quads = (a.rows + 3u) / 4u, qa = a.split >= a.rows ? quads : a.split / 4u;
    const uint32_t ga = a.grid_a, G = gridDim.x;
    const bool second = blockIdx.x >= ga;
    const float* const scale = second ? a.scale2 : a.scale;
    const float* const shift = second ? a.shift2 : a.shift;
    const uint32_t q0 = second ? qa + (blockIdx.x - ga) : blockIdx.x, qend = second ? quads : qa;
    const uint32_t qstep = second ? G - ga : ga;
#pragma unroll
    for (int j = 0; j < NV / 4; ++j) {
        const uint32_t k = threadIdx.x + 256u * j, c = 4u * k;
        const f32x4 z{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (!LN) vec_lds[kW][k] = c < a.dim ? ld4(a.w + c) : z;
        if (scale) vec_lds[kS][k] = c < a.dim ? 1.0f + ld4(scale + c) : z;
        if (shift) vec_lds[kH][k] = c < a.dim ? ld4(shift + c) : z;
    }
    __syncthreads();
    auto one_row = [&](uint32_t row) __attribute__((always_inline)) {
        const float* xr = a.x + (size_t)row * a.x_stride;
        f32x4 v[NV];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            v[i] = c < a.dim ? ld4(xr + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if constexpr (LN) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
            else s += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
        }
        s = wave_sum(s);
        float mean = 0.0f, r;
        if constexpr (LN) {
            mean = s / (float)a.dim;
            float qs = 0.0f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const uint32_t c = 4u * lane + 256u * i;
                if (c < a.dim) {
                    const f32x4 d = v[i] - mean;
                    qs += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
                }
            }
            qs = wave_sum(qs);
            r = 1.0f / __builtin_sqrtf(qs / (float)a.dim + a.eps);
        } else {
            r = 1.0f / __builtin_sqrtf(s / (float)a.dim + a.eps);
        }
        char* orow = (char*)a.out + (size_t)row * a.out_stride * (OT == kGgmlF32 ? 4u : 2u);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            if (c >= a.dim) continue;
            f32x4 y;
            if constexpr (LN) y = (v[i] - mean) * r;
            else y = (v[i] * r) * vec_lds[kW][lane + 64u * i];
            if (scale) y = y * vec_lds[kS][lane + 64u * i];
            if (shift) y = y + vec_lds[kH][lane + 64u * i];
            store4<OT>(orow, c, y);
        }
    };
    if constexpr (LN) {  // one group per workgroup: no loop (it cost 19 registers and a round)
        const uint32_t row = q0 * 4u + (threadIdx.x >> 6);
        if (q0 < qend && row < a.rows) one_row(row);
    } else {
        for (uint32_t q = q0; q < qend; q += qstep) {
            const uint32_t row = q * 4u + (threadIdx.x >> 6);
            if (row >= a.rows) break;  // the last group only
            one_row(row);
        }
    }
}

// --- qkv_heads ---------------------------------------------------------------
// Workgroup (row r, slot s in {Q, K, V}); each wave walks heads h = wave,
// wave + 4, ...; lane l owns the RoPE pair (2l, 2l+1) of a 128-wide head.
//   x   = src[r, s*H*128 + h*128 + 2l .. +1]                (f32)
//   Q,K: x = x * (1 / sqrt(sum_head(x^2) / 128 + eps)) * w  (batch_head_norm,
//        zimage.slang:624-667), when the slot's weight is given
//   Q,K: (x0, x1) -> (x0*c - x1*s, x0*s + x1*c) with c, s = cos/sin[t, l]
//        (mrope.slang:45-53), when tables are given; t = dst_row0 + r
//   dst_s[h, t, 2l .. +1] = x                               (transpose_heads
//        direction 0, zimage.slang:576-601, into the joint sequence at row t)

template <uint32_t OT>
__global__ void __launch_bounds__(256) qkv_heads_kernel(QkvHeadsArgs a) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t r = blockIdx.x, slot = blockIdx.y;
    const uint32_t t = a.dst_row0 + r;
    const uint32_t hd = a.n_heads * 128u;
    const float* src = a.src + (size_t)r * a.src_stride + slot * hd + 2u * lane;
    const float* w = slot == 0 ? a.q_norm : (slot == 1 ? a.k_norm : nullptr);
    void* dst = slot == 0 ? a.q : (slot == 1 ? a.k : a.v);
    const bool rope = slot < 2 && a.rope_cos != nullptr;
    float c = 1.0f, sn = 0.0f;
    if (rope) {
        c = a.rope_cos[(size_t)t * 64u + lane];
        sn = a.rope_sin[(size_t)t * 64u + lane];
    }
    float w0 = 1.0f, w1 = 1.0f;
    if (w) {
        w0 = w[2u * lane];
        w1 = w[2u * lane + 1u];
    }
    // the wave's heads h = wave, wave + 4, ... are all requested before the
    // first is processed (up to kHB at a time), so their loads overlap
    constexpr uint32_t kHB = 8;
    for (uint32_t h0 = wave; h0 < a.n_heads; h0 += 4u * kHB) {
        f32x2 xv[kHB];
#pragma unroll
        for (uint32_t j = 0; j < kHB; ++j) {
            const uint32_t h = h0 + 4u * j;
            xv[j] = h < a.n_heads ? *(const f32x2*)(src + h * 128u) : f32x2{0.0f, 0.0f};
        }
#pragma unroll
        for (uint32_t j = 0; j < kHB; ++j) {
            const uint32_t h = h0 + 4u * j;
            if (h >= a.n_heads) break;  // uniform over the wave
            float x0 = xv[j].x, x1 = xv[j].y;
            if (w) {
                const float ss = wave_sum(x0 * x0 + x1 * x1);
                const float rms = 1.0f / __builtin_sqrtf(ss / 128.0f + a.eps);
                x0 = (x0 * rms) * w0;
                x1 = (x1 * rms) * w1;
            }
            if (rope) {
                const float y0 = x0 * c - x1 * sn;
                const float y1 = x0 * sn + x1 * c;
                x0 = y0;
                x1 = y1;
            }
            store2<OT>(dst, ((size_t)h * a.dst_seq + t) * 128u + 2u * lane, x0, x1);
        }
    }
}

// --- residual ----------------------------------------------------------------
// h[r, d] += g(d) * y[r, d] with y = x or, when norm_w is given, the RMS
// normalised x (batch_rmsnorm, zimage.slang:465-500), and
//   gate == null:      g = 1                     (residual_add, diffusion.slang:1713-1716)
//   linear gate:       g = gate[d]               (gated_residual_linear, zimage.slang:414-424)
//   tanh gate:         clamp(1 * tanh(gate[d]) * y, +-1e10)
//                                                (gated_residual, zimage.slang:395-410,
//                                                 scale 1, no clip threshold)

template <bool NORM, bool TANH, int NV>
__global__ void __launch_bounds__(256) residual_kernel(ResidualArgs a) {
    // the norm weights and the gate (tanh(gate) for TANH), staged once per
    // workgroup (element 4k .. 4k+3 at k); a persistent grid of two
    // workgroups per CU walks the groups of four rows
    __shared__ f32x4 vec_lds[2][NV * 64];
    const uint32_t lane = threadIdx.x & 63u;
    if (NORM || a.gate) {  // uniform over the workgroup
#pragma unroll
        for (int j = 0; j < NV / 4; ++j) {
            const uint32_t k = threadIdx.x + 256u * j, c = 4u * k;
            if constexpr (NORM) vec_lds[0][k] = c < a.dim ? ld4(a.norm_w + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (a.gate) {
                const f32x4 g = c < a.dim ? ld4(a.gate + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (TANH) vec_lds[1][k] = f32x4{tanhf(g.x), tanhf(g.y), tanhf(g.z), tanhf(g.w)};
                else vec_lds[1][k] = g;
            }
        }
        __syncthreads();
    }
    const uint32_t quads = (a.rows + 3u) / 4u;
    for (uint32_t q = blockIdx.x; q < quads; q += gridDim.x) {
        const uint32_t row = q * 4u + (threadIdx.x >> 6);
        if (row >= a.rows) break;  // the last group only
        const float* xr = a.x + (size_t)row * a.x_stride;
        float* hr = a.h + (size_t)row * a.h_stride;
        f32x4 v[NV], hv[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            v[i] = c < a.dim ? ld4(xr + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            hv[i] = c < a.dim ? ld4(hr + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        float s = 0.0f;
        if constexpr (NORM) {
#pragma unroll
            for (int i = 0; i < NV; ++i)
                s += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
        }
        float rms = 1.0f;
        if constexpr (NORM) rms = 1.0f / __builtin_sqrtf(wave_sum(s) / (float)a.dim + a.eps);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            if (c >= a.dim) continue;
            f32x4 y = v[i];
            if constexpr (NORM) y = (y * rms) * vec_lds[0][lane + 64u * i];
            if (a.gate) {
                const f32x4 g = vec_lds[1][lane + 64u * i];
                if constexpr (TANH) {
                    const f32x4 tg = g;
                    y = (1.0f * tg) * y;
                    y = __builtin_elementwise_min(__builtin_elementwise_max(y, f32x4(-1e10f)), f32x4(1e10f));
                } else {
                    y = g * y;
                }
            }
            *(f32x4*)(hr + c) = hv[i] + y;
        }
    }
}

// The same update, then the updated row's RMSNorm (weight next_w) * (1 +
// next_scale) + next_shift into out: the post-norm residual of one half of
// a Z-Image block and the next half's pre-norm (dit.c3:1495-1503 then
// 1545-1554) in one pass over the rows. The arithmetic is residual_kernel's,
// then row_norm_kernel's (RMS) on the updated row in registers, in the same
// order, so the results equal the two launches bit for bit.
template <bool NORM, bool TANH, uint32_t OT, int NV>
__global__ void __launch_bounds__(256) residual_norm_kernel(ResidualArgs a) {
    // x's norm weights, the gate (tanh(gate) for TANH), next_w and
    // 1 + next_scale, staged once per workgroup; the workgroups then take
    // groups of four rows in turn (a persistent grid of two per CU: one
    // workgroup of four rows each would run 4352 rows in 2.1 rounds of
    // three, and stage the vectors 1088 times)
    __shared__ f32x4 vec_lds[4][NV * 64];
#pragma unroll
    for (int j = 0; j < NV / 4; ++j) {
        const uint32_t k = threadIdx.x + 256u * j, c = 4u * k;
        const f32x4 z{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (NORM) vec_lds[0][k] = c < a.dim ? ld4(a.norm_w + c) : z;
        if (a.gate) {
            const f32x4 g = c < a.dim ? ld4(a.gate + c) : z;
            if constexpr (TANH) vec_lds[1][k] = f32x4{tanhf(g.x), tanhf(g.y), tanhf(g.z), tanhf(g.w)};
            else vec_lds[1][k] = g;
        }
        vec_lds[2][k] = c < a.dim ? ld4(a.next_w + c) : z;
        if (a.next_scale) vec_lds[3][k] = c < a.dim ? 1.0f + ld4(a.next_scale + c) : z;
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t quads = (a.rows + 3u) / 4u;
    for (uint32_t q = blockIdx.x; q < quads; q += gridDim.x) {
        const uint32_t row = q * 4u + (threadIdx.x >> 6);
        if (row >= a.rows) break;  // the last quad only: no later one for this wave
        const float* xr = a.x + (size_t)row * a.x_stride;
        float* hr = a.h + (size_t)row * a.h_stride;
        f32x4 v[NV], hv[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            v[i] = c < a.dim ? ld4(xr + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            hv[i] = c < a.dim ? ld4(hr + c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        float s = 0.0f;
        if constexpr (NORM) {
#pragma unroll
            for (int i = 0; i < NV; ++i)
                s += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
        }
        float rms = 1.0f;
        if constexpr (NORM) rms = 1.0f / __builtin_sqrtf(wave_sum(s) / (float)a.dim + a.eps);
        float s2 = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            if (c < a.dim) {
                f32x4 y = v[i];
                if constexpr (NORM) y = (y * rms) * vec_lds[0][lane + 64u * i];
                if (a.gate) {
                    const f32x4 g = vec_lds[1][lane + 64u * i];
                    if constexpr (TANH) {
                        y = (1.0f * g) * y;
                        y = __builtin_elementwise_min(__builtin_elementwise_max(y, f32x4(-1e10f)), f32x4(1e10f));
                    } else {
                        y = g * y;
                    }
                }
                hv[i] = hv[i] + y;
                *(f32x4*)(hr + c) = hv[i];
            }
            s2 += (hv[i].x * hv[i].x + hv[i].y * hv[i].y) + (hv[i].z * hv[i].z + hv[i].w * hv[i].w);
        }
        const float r2 = 1.0f / __builtin_sqrtf(wave_sum(s2) / (float)a.dim + a.next_eps);
        char* orow = (char*)a.out + (size_t)row * a.out_stride * (OT == kGgmlF32 ? 4u : 2u);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = 4u * lane + 256u * i;
            if (c >= a.dim) continue;
            f32x4 y = (hv[i] * r2) * vec_lds[2][lane + 64u * i];
            if (a.next_scale) y = y * vec_lds[3][lane + 64u * i];
            if (a.next_shift) y = y + ld4(a.next_shift + c);
            store4<OT>(orow, c, y);
        }
    }
}

// --- act_cols ----------------------------------------------------------------
// dst[r, dst_col + c] = f(src[r, src_col + c] (, src[r, src2_col + c])) for
// c < cols, four columns per thread:
//   copy:      x
//   silu:      x / (1 + exp(-x))                              (diffusion.slang:1082-1086)
//   gelu:      0.5*x*(1 + tanh(0.7978845608*(x + 0.044715*x*x*x)))
//                                                             (diffusion.slang:1103-1107)
//   silu_mul:  silu(x) * src[r, src2_col + c]                 (silu then elemwise_mul,
//                                                              diffusion.slang:1733-1736)

__device__ __forceinline__ float silu_ref(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float gelu_ref(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

template <int ACT, uint32_t OT>
__global__ void __launch_bounds__(256) act_cols_kernel(ActColsArgs a) {
    const uint32_t nbc = (a.cols / 4u + 255u) / 256u;  // workgroups per row
    const uint32_t r = blockIdx.x / nbc;
    const uint32_t c = ((blockIdx.x % nbc) * 256u + threadIdx.x) * 4u;
    if (c >= a.cols) return;
    const float* sr = a.src + (size_t)r * a.src_stride;
    f32x4 x = ld4(sr + a.src_col + c);
    if constexpr (ACT == kActSilu || ACT == kActSiluMul) {
        x = f32x4{silu_ref(x.x), silu_ref(x.y), silu_ref(x.z), silu_ref(x.w)};
        if constexpr (ACT == kActSiluMul) x = x * ld4(sr + a.src2_col + c);
    } else if constexpr (ACT == kActGelu) {
        x = f32x4{gelu_ref(x.x), gelu_ref(x.y), gelu_ref(x.z), gelu_ref(x.w)};
    }
    store4<OT>(a.dst, (size_t)r * a.dst_stride + a.dst_col + c, x);
}

// --- timestep embedding, (un)patchify ----------------------------------------

// out[i] = cos(t * f_i) for i < dim/2, sin(t * f_{i - dim/2}) above, with
// f_j = exp(-ln(10000) * j / (dim/2))  (dit_timestep_embed, zimage.slang:294-307).
__global__ void __launch_bounds__(256) timestep_embed_kernel(float* out, uint32_t dim, float t) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t half = dim / 2u;
    if (i >= dim) return;
    const uint32_t j = i < half ? i : i - half;
    const float freq = expf(-logf(10000.0f) * (float)j / (float)half);
    out[i] = i < half ? cosf(t * freq) : sinf(t * freq);
}

// [C, H, W] -> [n_patches, C*ps*ps] with element e = (py*ps + px)*C + c of
// patch (H/ps row-major) (patchify, zimage.slang:24-51); one thread per output.
template <uint32_t OT>
__global__ void __launch_bounds__(256) patchify_kernel(const float* in, void* out, uint32_t C, uint32_t H,
                                                        uint32_t W, uint32_t ps) {
    const uint32_t pd = C * ps * ps, pw = W / ps, n = (H / ps) * pw * pd;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const uint32_t p = i / pd, e = i % pd;
    const uint32_t py = e / (ps * C), px = (e % (ps * C)) / C, c = e % C;
    const uint32_t ih = (p / pw) * ps + py, iw = (p % pw) * ps + px;
    const float v = in[((size_t)c * H + ih) * W + iw];
    if constexpr (OT == kGgmlF32) ((float*)out)[i] = v;
    else if constexpr (OT == kGgmlF16) ((_Float16*)out)[i] = (_Float16)v;
    else ((__bf16*)out)[i] = (__bf16)v;
}

// The inverse permutation, f32 (unpatchify, zimage.slang:69-93).
__global__ void __launch_bounds__(256) unpatchify_kernel(const float* in, float* out, uint32_t C, uint32_t H,
                                                          uint32_t W, uint32_t ps) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= C * H * W) return;
    const uint32_t c = i / (H * W), rem = i % (H * W), h = rem / W, w = rem % W;
    const uint32_t p = (h / ps) * (W / ps) + w / ps;
    const uint32_t e = (h % ps) * ps * C + (w % ps) * C + c;
    out[i] = in[(size_t)p * C * ps * ps + e];
}

// --- dispatch helpers ----------------------------------------------------------

template <uint32_t OT>
hipError_t launch_row_norm_t(RowNormArgs a, bool ln, hipStream_t st) {
    // LayerNorm: one workgroup per group of four rows; RMSNorm: two per CU.
    // The workgroups are split between the sides in proportion to their
    // groups (each side at least one when it has rows).
    const uint32_t quads = (a.rows + 3u) / 4u, qa = a.split >= a.rows ? quads : a.split / 4u, qb = quads - qa;
    const uint32_t G = ln ? quads : persistent_grid(a.rows, a.grid_cus);
    uint32_t ga = qb == 0 ? G : qa == 0 ? 0u : (uint32_t)(((uint64_t)G * qa + quads / 2u) / quads);
    if (qa > 0 && ga == 0) ga = 1;
    if (qb > 0 && ga == G) ga = G - 1u;
    a.grid_a = ga;
    const dim3 grid(G), block(256);
    const uint32_t nv = (a.dim + 255u) / 256u;
#define LLMR_ROW_NORM(NVV)                                                                              \
    if (nv <= NVV) {                                                                                    \
        if (ln) hipLaunchKernelGGL((row_norm_kernel<true, OT, NVV>), grid, block, 0, st, a);            \
        else hipLaunchKernelGGL((row_norm_kernel<false, OT, NVV>), grid, block, 0, st, a);              \
        return hipGetLastError();                                                                       \
    }
    LLMR_ROW_NORM(4)
    LLMR_ROW_NORM(8)
    LLMR_ROW_NORM(12)
    LLMR_ROW_NORM(16)
    LLMR_ROW_NORM(32)
#undef LLMR_ROW_NORM
    return hipErrorInvalidValue;
}

template <bool NORM, bool TANH>
hipError_t launch_residual_t(const ResidualArgs& a, hipStream_t st) {
    const dim3 grid(persistent_grid(a.rows, a.grid_cus)), block(256);
    const uint32_t nv = (a.dim + 255u) / 256u;
    if (nv <= 4) hipLaunchKernelGGL((residual_kernel<NORM, TANH, 4>), grid, block, 0, st, a);
    else if (nv <= 8) hipLaunchKernelGGL((residual_kernel<NORM, TANH, 8>), grid, block, 0, st, a);
    else if (nv <= 16) hipLaunchKernelGGL((residual_kernel<NORM, TANH, 16>), grid, block, 0, st, a);
    else if (nv <= 32) hipLaunchKernelGGL((residual_kernel<NORM, TANH, 32>), grid, block, 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int ACT>
hipError_t launch_act_t(const ActColsArgs& a, uint32_t otype, hipStream_t st) {
    const dim3 grid((a.cols / 4u + 255u) / 256u * a.rows), block(256);
    switch (otype) {
        case kGgmlF32: hipLaunchKernelGGL((act_cols_kernel<ACT, kGgmlF32>), grid, block, 0, st, a); break;
        case kGgmlF16: hipLaunchKernelGGL((act_cols_kernel<ACT, kGgmlF16>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((act_cols_kernel<ACT, kGgmlBF16>), grid, block, 0, st, a); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_row_norm(const RowNormArgs& a, bool layernorm, uint32_t otype, hipStream_t st) {
    if (a.rows == 0) return hipSuccess;
    switch (otype) {
        case kGgmlF32: return launch_row_norm_t<kGgmlF32>(a, layernorm, st);
        case kGgmlF16: return launch_row_norm_t<kGgmlF16>(a, layernorm, st);
        default: return launch_row_norm_t<kGgmlBF16>(a, layernorm, st);
    }
}

hipError_t launch_qkv_heads(const QkvHeadsArgs& a, uint32_t otype, hipStream_t st) {
    if (a.rows == 0) return hipSuccess;
    const dim3 grid(a.rows, 3), block(256);
    switch (otype) {
        case kGgmlF32: hipLaunchKernelGGL(qkv_heads_kernel<kGgmlF32>, grid, block, 0, st, a); break;
        case kGgmlF16: hipLaunchKernelGGL(qkv_heads_kernel<kGgmlF16>, grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL(qkv_heads_kernel<kGgmlBF16>, grid, block, 0, st, a); break;
    }
    return hipGetLastError();
}

template <bool NORM, bool TANH, uint32_t OT>
hipError_t launch_residual_norm_t(const ResidualArgs& a, hipStream_t st) {
    const dim3 grid(persistent_grid(a.rows, a.grid_cus)), block(256);
    const uint32_t nv = (a.dim + 255u) / 256u;
    if (nv <= 4) hipLaunchKernelGGL((residual_norm_kernel<NORM, TANH, OT, 4>), grid, block, 0, st, a);
    else if (nv <= 8) hipLaunchKernelGGL((residual_norm_kernel<NORM, TANH, OT, 8>), grid, block, 0, st, a);
    else if (nv <= 16) hipLaunchKernelGGL((residual_norm_kernel<NORM, TANH, OT, 16>), grid, block, 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

template <uint32_t OT>
hipError_t launch_residual_norm_o(const ResidualArgs& a, bool tanh_gate, hipStream_t st) {
    if (a.norm_w)
        return tanh_gate ? launch_residual_norm_t<true, true, OT>(a, st) : launch_residual_norm_t<true, false, OT>(a, st);
    return tanh_gate ? launch_residual_norm_t<false, true, OT>(a, st) : launch_residual_norm_t<false, false, OT>(a, st);
}

hipError_t launch_residual_norm(const ResidualArgs& a, bool tanh_gate, uint32_t otype, hipStream_t st) {
    if (a.rows == 0) return hipSuccess;
    switch (otype) {
        case kGgmlF32: return launch_residual_norm_o<kGgmlF32>(a, tanh_gate, st);
        case kGgmlF16: return launch_residual_norm_o<kGgmlF16>(a, tanh_gate, st);
        default: return launch_residual_norm_o<kGgmlBF16>(a, tanh_gate, st);
    }
}

hipError_t launch_residual(const ResidualArgs& a, bool tanh_gate, hipStream_t st) {
    if (a.rows == 0) return hipSuccess;
    if (a.norm_w) return tanh_gate ? launch_residual_t<true, true>(a, st) : launch_residual_t<true, false>(a, st);
    return tanh_gate ? launch_residual_t<false, true>(a, st) : launch_residual_t<false, false>(a, st);
}

hipError_t launch_act_cols(const ActColsArgs& a, int act, uint32_t otype, hipStream_t st) {
    if (a.rows == 0 || a.cols == 0) return hipSuccess;
    switch (act) {
        case kActCopy: return launch_act_t<kActCopy>(a, otype, st);
        case kActSilu: return launch_act_t<kActSilu>(a, otype, st);
        case kActGelu: return launch_act_t<kActGelu>(a, otype, st);
        default: return launch_act_t<kActSiluMul>(a, otype, st);
    }
}

hipError_t launch_timestep_embed(float* out, uint32_t dim, float t, hipStream_t st) {
    hipLaunchKernelGGL(timestep_embed_kernel, dim3((dim + 255u) / 256u), dim3(256), 0, st, out, dim, t);
    return hipGetLastError();
}

hipError_t launch_patchify(const float* in, void* out, uint32_t otype, uint32_t C, uint32_t H, uint32_t W,
                           uint32_t ps, hipStream_t st) {
    const uint32_t n = C * H * W;
    const dim3 grid((n + 255u) / 256u), block(256);
    switch (otype) {
        case kGgmlF32: hipLaunchKernelGGL(patchify_kernel<kGgmlF32>, grid, block, 0, st, in, out, C, H, W, ps); break;
        case kGgmlF16: hipLaunchKernelGGL(patchify_kernel<kGgmlF16>, grid, block, 0, st, in, out, C, H, W, ps); break;
        default: hipLaunchKernelGGL(patchify_kernel<kGgmlBF16>, grid, block, 0, st, in, out, C, H, W, ps); break;
    }
    return hipGetLastError();
}

hipError_t launch_unpatchify(const float* in, float* out, uint32_t C, uint32_t H, uint32_t W, uint32_t ps,
                             hipStream_t st) {
    const uint32_t n = C * H * W;
    hipLaunchKernelGGL(unpatchify_kernel, dim3((n + 255u) / 256u), dim3(256), 0, st, in, out, C, H, W, ps);
    return hipGetLastError();
}

}  // namespace llmr
