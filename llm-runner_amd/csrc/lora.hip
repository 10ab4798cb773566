// lora.hip - LoRA adapters on the DiT linears, in the reference's two forms:
//
//  * the runtime two-hop correction appended to a base batch_matmul output
//    (dispatch_lora_correction, dit.c3:1319-1364): hop 1 scratch = x . A^T
//    (batch_matmul_simple, llm.slang:1146-1180), hop 2 output += scale *
//    scratch . B^T (batch_matmul_add_scaled, llm.slang:1262-1294);
//  * the load-time merge into a Q8_0 weight with per-block requantization
//    (q8_lora_merge, llm.slang:1337-1420; host merge_one_site,
//    lora_merge.c3:36-73).
//
// The dot products are fused multiply-adds (the reference's `partial += a *
// b` leaves contraction to its shader compiler), every other f32 operation
// rounds where the reference's source writes it, and every sum is formed in
// the reference's order, so the results are bit-identical to the CPU
// restatement: hop 1's sums as a 256-thread workgroup forms them (strided
// partials, then the tree), hop 2's and the merge's in rank order.
//
// Work layout (MI355X): hop 1 gives each workgroup 4 tokens x 8 ranks per
// pass (A is read once per 4 tokens instead of once per (token, rank) sum),
// its k loop unrolled for loads in flight and a small LDS tree for several
// workgroups per CU; hop 2 gives each workgroup 256 output features x 64
// tokens, so B is read once per 64 tokens. Both are
// bandwidth-bound: the dominant traffic is hop 2's read-modify-write of the
// f32 output.
#include <hip/hip_runtime.h>

#include "llmr_device.h"
#include "llmr_internal.h"

#include <type_traits>

#pragma clang fp contract(off)

namespace llmr {
namespace {

constexpr uint32_t kDownTokens = 4;   // tokens per hop-1 workgroup
constexpr uint32_t kDownRanks = 8;    // rank outputs per hop-1 pass
constexpr uint32_t kDownTree = 32;    // sums per LDS tree round
constexpr uint32_t kUpTokens = 32;    // tokens per hop-2 workgroup
constexpr uint32_t kUpChunk = 32;     // ranks per hop-2 LDS pass

template <uint32_t XT>
__device__ __forceinline__ float load_act(const void* X, uint64_t i) {
    if constexpr (XT == kGgmlF32) {
        return ((const float*)X)[i];
    } else if constexpr (XT == kGgmlBF16) {
        return __uint_as_float((uint32_t)((const uint16_t*)X)[i] << 16);
    } else {
        return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)X)[i]);
    }
}

// scratch[s, r] = sum_k A[r, k] * X[s, k]: thread gi accumulates k = gi,
// gi + 256, ... in order, then the tree s = 128 .. 1 of batch_matmul_simple.
template <uint32_t XT>
__global__ void __launch_bounds__(256) lora_down_kernel(const float* __restrict__ A, const void* __restrict__ X,
                                                         float* __restrict__ scratch, uint32_t rank, uint32_t in_dim,
                                                         uint32_t seq_len) {
    constexpr uint32_t Q = kDownTokens * kDownRanks;  // sums per pass, reduced kDownTree at a time
    __shared__ float red[kDownTree][256];
    const uint32_t gi = threadIdx.x;
    const uint32_t s0 = blockIdx.x * kDownTokens;
    for (uint32_t r0 = 0; r0 < rank; r0 += kDownRanks) {
        float part[kDownTokens][kDownRanks];
#pragma unroll
        for (uint32_t t = 0; t < kDownTokens; t++)
#pragma unroll
            for (uint32_t r = 0; r < kDownRanks; r++) part[t][r] = 0.0f;
#pragma unroll 4
        for (uint32_t k = gi; k < in_dim; k += 256u) {
            float x[kDownTokens];
#pragma unroll
            for (uint32_t t = 0; t < kDownTokens; t++)
                x[t] = s0 + t < seq_len ? load_act<XT>(X, (uint64_t)(s0 + t) * in_dim + k) : 0.0f;
#pragma unroll
            for (uint32_t r = 0; r < kDownRanks; r++) {
                const float a = r0 + r < rank ? A[(uint64_t)(r0 + r) * in_dim + k] : 0.0f;
#pragma unroll
                for (uint32_t t = 0; t < kDownTokens; t++) part[t][r] = __builtin_fmaf(a, x[t], part[t][r]);
            }
        }
#pragma unroll
        for (uint32_t h = 0; h < Q / kDownTree; h++) {
#pragma unroll
            for (uint32_t q = 0; q < kDownTree; q++)
                red[q][gi] = part[(h * kDownTree + q) / kDownRanks][(h * kDownTree + q) % kDownRanks];
            __syncthreads();
#pragma unroll
            for (uint32_t ls = 7; ls < 8; ls--) {  // s = 2^ls = 128, 64, ..., 1
                const uint32_t s = 1u << ls;
                for (uint32_t item = gi; item < kDownTree * s; item += 256u) {
                    const uint32_t q = item >> ls, i = item & (s - 1u);
                    red[q][i] += red[q][i + s];
                }
                __syncthreads();
            }
            if (gi < kDownTree) {
                const uint32_t qq = h * kDownTree + gi, t = qq / kDownRanks, r = qq % kDownRanks;
                if (s0 + t < seq_len && r0 + r < rank) scratch[(uint64_t)(s0 + t) * rank + r0 + r] = red[gi][0];
            }
            __syncthreads();  // red is rewritten by the next half
        }
    }
}

// out[s * out_dim + row_offset + o] += scale * sum_r B[(wro + o) * rank + r] *
// scratch[s * rank + r] for o < b_rows, the sum in rank order. A workgroup
// takes 512 outputs (thread gi: o0 + gi and o0 + 256 + gi) x kUpTokens
// tokens; B's rows for its outputs pass through LDS in chunks of kUpChunk
// ranks (read coalesced, stored transposed with a pad so thread gi reads its
// columns without bank conflicts) and stay in registers while the tokens'
// scratch rows are read as 16-byte broadcasts.
__global__ void __launch_bounds__(256) lora_up_kernel(const float* __restrict__ B, const float* __restrict__ scratch,
                                                       float* __restrict__ out, uint32_t rank, uint32_t out_dim,
                                                       uint32_t seq_len, float scale, uint32_t row_offset,
                                                       uint32_t weight_row_offset, uint32_t b_rows) {
    __shared__ __attribute__((aligned(16))) float sc[kUpTokens][kUpChunk];
    __shared__ float bs[kUpChunk][513];
    const uint32_t gi = threadIdx.x;
    const uint32_t o0 = blockIdx.x * 512u, s0 = blockIdx.y * kUpTokens;
    const uint32_t nt = min(kUpTokens, seq_len - s0), no = min(512u, b_rows - o0);
    float acc[2][kUpTokens];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++)
#pragma unroll
        for (uint32_t t = 0; t < kUpTokens; t++) acc[h][t] = 0.0f;
    for (uint32_t r0 = 0; r0 < rank; r0 += kUpChunk) {
        const uint32_t nr = min(kUpChunk, rank - r0);
        if (nr == kUpChunk && rank % 4u == 0u) {
            // whole chunks: 16-byte loads (B rows and scratch rows are 16-byte
            // aligned: rank % 4 == 0), indices by shifts
            for (uint32_t i = gi; i < no * (kUpChunk / 4u); i += 256u) {
                const uint32_t o = i >> 3, r = (i & 7u) * 4u;
                const f32x4 v = *(const f32x4*)(B + (uint64_t)(weight_row_offset + o0 + o) * rank + r0 + r);
                bs[r][o] = v.x;
                bs[r + 1][o] = v.y;
                bs[r + 2][o] = v.z;
                bs[r + 3][o] = v.w;
            }
            for (uint32_t i = gi; i < nt * (kUpChunk / 4u); i += 256u) {
                const uint32_t t = i >> 3, r = (i & 7u) * 4u;
                *(f32x4*)&sc[t][r] = *(const f32x4*)(scratch + (uint64_t)(s0 + t) * rank + r0 + r);
            }
        } else {
            for (uint32_t i = gi; i < no * nr; i += 256u) {
                const uint32_t o = i / nr, r = i % nr;
                bs[r][o] = B[(uint64_t)(weight_row_offset + o0 + o) * rank + r0 + r];
            }
            for (uint32_t i = gi; i < nt * nr; i += 256u) {
                const uint32_t t = i / nr, r = i % nr;
                sc[t][r] = scratch[(uint64_t)(s0 + t) * rank + r0 + r];
            }
        }
        __syncthreads();
        if (nr == kUpChunk) {
            float bv[2][kUpChunk];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++)
#pragma unroll
                for (uint32_t r = 0; r < kUpChunk; r++) bv[h][r] = bs[r][h * 256u + gi];
#pragma unroll
            for (uint32_t t = 0; t < kUpTokens; t++) {
                float a0 = acc[0][t], a1 = acc[1][t];
#pragma unroll
                for (uint32_t r = 0; r < kUpChunk; r++) {
                    const float sv = sc[t][r];
                    a0 = __builtin_fmaf(bv[0][r], sv, a0);
                    a1 = __builtin_fmaf(bv[1][r], sv, a1);
                }
                acc[0][t] = a0;
                acc[1][t] = a1;
            }
        } else {  // the last, partial chunk of ranks
            for (uint32_t r = 0; r < nr; r++) {
                const float b0 = bs[r][gi], b1 = bs[r][256u + gi];
#pragma unroll
                for (uint32_t t = 0; t < kUpTokens; t++) {
                    acc[0][t] = __builtin_fmaf(b0, sc[t][r], acc[0][t]);
                    acc[1][t] = __builtin_fmaf(b1, sc[t][r], acc[1][t]);
                }
            }
        }
        __syncthreads();  // bs and sc are refilled by the next chunk
    }
    // (columns past b_rows and tokens past seq_len are neither read nor
    // written; their acc entries hold LDS leftovers). All of the thread's
    // output reads are issued before any write, so their latencies overlap
    // instead of one read-modify-write waiting per token.
    float* const ybase = out + (uint64_t)s0 * out_dim + row_offset + o0 + gi;
    float yv[2][kUpTokens];
#pragma unroll
    for (uint32_t h = 0; h < 2; h++)
#pragma unroll
        for (uint32_t t = 0; t < kUpTokens; t++)
            yv[h][t] = (h * 256u + gi < no && t < nt) ? ybase[(uint64_t)t * out_dim + h * 256u] : 0.0f;
#pragma unroll
    for (uint32_t h = 0; h < 2; h++)
#pragma unroll
        for (uint32_t t = 0; t < kUpTokens; t++)
            if (h * 256u + gi < no && t < nt) ybase[(uint64_t)t * out_dim + h * 256u] = yv[h][t] + scale * acc[h][t];
}

// Hop 2 for ranks up to RK (8, 16 or 32; rank % 4 == 0): thread gi owns
// output column o0 + gi, whose B row (rank floats) stays in registers for
// the workgroup's kUpRegSpan tokens; the tokens' scratch rows go through LDS
// in blocks of kUpRegTokens (broadcast reads), the block's output values are
// read before its sums. Same arithmetic as lora_up_kernel: the sum over
// ranks in rank order from 0, then y + scale * sum. Its LDS footprint is
// 2 KiB (lora_up_kernel's 70 KiB held two workgroups per CU), so enough
// workgroups share a CU to overlap their output reads and writes with the
// FMAs of others.
constexpr uint32_t kUpRegTokens = 16;
constexpr uint32_t kUpRegSpan = 128;
template <uint32_t RK>
__global__ void __launch_bounds__(256) lora_up_reg_kernel(const float* __restrict__ B,
                                                           const float* __restrict__ scratch, float* __restrict__ out,
                                                           uint32_t rank, uint32_t out_dim, uint32_t seq_len,
                                                           float scale, uint32_t row_offset, uint32_t weight_row_offset,
                                                           uint32_t b_rows) {
    __shared__ __attribute__((aligned(16))) float sc[kUpRegTokens][RK];
    const uint32_t gi = threadIdx.x, o = blockIdx.x * 256u + gi;
    const uint32_t s_begin = blockIdx.y * kUpRegSpan, s_end = min(seq_len, s_begin + kUpRegSpan);
    const bool live = o < b_rows;
    const uint32_t q = rank / 4u;  // 16-byte pieces of a rank row
    float bv[RK];
#pragma unroll
    for (uint32_t r = 0; r < RK; r += 4) {
        const f32x4 v = live && r < rank ? *(const f32x4*)(B + (uint64_t)(weight_row_offset + o) * rank + r)
                                         : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        bv[r] = v.x;
        bv[r + 1] = v.y;
        bv[r + 2] = v.z;
        bv[r + 3] = v.w;
    }
    float* const ycol = out + row_offset + o;
    for (uint32_t s0 = s_begin; s0 < s_end; s0 += kUpRegTokens) {
        const uint32_t nt = min(kUpRegTokens, s_end - s0);
        for (uint32_t i = gi; i < nt * q; i += 256u) {
            const uint32_t t = i / q, r = 4u * (i % q);
            *(f32x4*)&sc[t][r] = *(const f32x4*)(scratch + (uint64_t)(s0 + t) * rank + r);
        }
        __syncthreads();
        float yv[kUpRegTokens];
#pragma unroll
        for (uint32_t t = 0; t < kUpRegTokens; t++)
            yv[t] = live && t < nt ? ycol[(uint64_t)(s0 + t) * out_dim] : 0.0f;
#pragma unroll
        for (uint32_t t = 0; t < kUpRegTokens; t++) {
            float a = 0.0f;
#pragma unroll
            for (uint32_t r = 0; r < RK; r++)
                if (r < rank) a = __builtin_fmaf(bv[r], sc[t][r], a);
            if (live && t < nt) ycol[(uint64_t)(s0 + t) * out_dim] = yv[t] + scale * a;
        }
        __syncthreads();  // sc is refilled by the next block
    }
}

// One 256-element chunk (8 Q8_0 blocks = 272 bytes) of LoRA row blockIdx.y:
// thread gi owns element k = 256 blockIdx.x + gi.
__global__ void __launch_bounds__(256) q8_lora_merge_kernel(uint8_t* __restrict__ base, const float* __restrict__ A,
                                                             const float* __restrict__ B, uint32_t in_dim,
                                                             uint32_t dst_row_offset, uint32_t rank, float scale) {
    __shared__ float brow[kMaxLoraRank];
    __shared__ float amax[256];
    const uint32_t gi = threadIdx.x, j = blockIdx.y;
    const uint32_t blk = gi / 32u, e = gi % 32u;
    const uint32_t k = blockIdx.x * 256u + gi;
    for (uint32_t r = gi; r < rank; r += 256u) brow[r] = B[(uint64_t)j * rank + r];
    uint8_t* const b = base + (uint64_t)(dst_row_offset + j) * (in_dim / 32u) * 34u +
                       (uint64_t)(blockIdx.x * 8u + blk) * 34u;
    const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    const float base_val = d * (float)(int8_t)b[2 + e];
    __syncthreads();
    float delta = 0.0f;
    for (uint32_t r = 0; r < rank; r++) delta = __builtin_fmaf(brow[r], A[(uint64_t)r * in_dim + k], delta);
    delta *= scale;
    const float u = base_val + delta;
    amax[gi] = fabsf(u);
    __syncthreads();
    for (uint32_t s = 16; s > 0; s >>= 1) {
        if (e < s) amax[gi] = fmaxf(amax[gi], amax[gi + s]);
        __syncthreads();
    }
    float dn = amax[blk * 32u] / 127.0f;
    if (dn < 1e-8f) dn = 1e-8f;
    const float qf = u / dn;
    int q = qf >= 0.0f ? (int)(qf + 0.5f) : (int)(qf - 0.5f);
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    b[2 + e] = (uint8_t)(int8_t)q;  // every read of this chunk precedes the barriers above
    if (e == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)dn);
        b[0] = (uint8_t)(h & 0xffu);
        b[1] = (uint8_t)(h >> 8);
    }
}

}  // namespace

hipError_t launch_lora_correction(const float* A, const float* B, uint32_t rank, float scale, float* scratch,
                                  const void* x, uint32_t xtype, float* out, uint32_t in_dim, uint32_t out_dim,
                                  uint32_t seq_len, uint32_t b_rows, uint32_t row_offset, uint32_t weight_row_offset,
                                  hipStream_t st) {
    if (rank == 0 || seq_len == 0) return hipSuccess;
    const dim3 gd((seq_len + kDownTokens - 1) / kDownTokens);
    switch (xtype) {
        case kGgmlF32:
            hipLaunchKernelGGL(lora_down_kernel<kGgmlF32>, gd, dim3(256), 0, st, A, x, scratch, rank, in_dim, seq_len);
            break;
        case kGgmlF16:
            hipLaunchKernelGGL(lora_down_kernel<kGgmlF16>, gd, dim3(256), 0, st, A, x, scratch, rank, in_dim, seq_len);
            break;
        default:
            hipLaunchKernelGGL(lora_down_kernel<kGgmlBF16>, gd, dim3(256), 0, st, A, x, scratch, rank, in_dim,
                               seq_len);
            break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || b_rows == 0) return e;
    if (rank <= 32u && rank % 4u == 0u) {
        const dim3 gr((b_rows + 255u) / 256u, (seq_len + kUpRegSpan - 1) / kUpRegSpan);
        auto go = [&](auto rk) {
            hipLaunchKernelGGL(lora_up_reg_kernel<decltype(rk)::value>, gr, dim3(256), 0, st, B,
                               (const float*)scratch, out, rank, out_dim, seq_len, scale, row_offset,
                               weight_row_offset, b_rows);
        };
        if (rank <= 8u) go(std::integral_constant<uint32_t, 8>{});
        else if (rank <= 16u) go(std::integral_constant<uint32_t, 16>{});
        else go(std::integral_constant<uint32_t, 32>{});
        return hipGetLastError();
    }
    const dim3 gu((b_rows + 511u) / 512u, (seq_len + kUpTokens - 1) / kUpTokens);
    hipLaunchKernelGGL(lora_up_kernel, gu, dim3(256), 0, st, B, (const float*)scratch, out, rank, out_dim, seq_len,
                       scale, row_offset, weight_row_offset, b_rows);
    return hipGetLastError();
}

hipError_t launch_q8_lora_merge(void* base, const float* A, const float* B, uint32_t in_dim, uint32_t b_rows,
                                uint32_t dst_row_offset, uint32_t rank, float scale, hipStream_t st) {
    if (b_rows == 0) return hipSuccess;
    hipLaunchKernelGGL(q8_lora_merge_kernel, dim3(in_dim / 256u, b_rows), dim3(256), 0, st, (uint8_t*)base, A, B,
                       in_dim, dst_row_offset, rank, scale);
    return hipGetLastError();
}

}  // namespace llmr
