// gemv_q.hip - Q4_K dequant-GEMM for a handful of tokens (M <= 4): the
// modulation and timestep projections of a DiT step (M = 1) stream a whole
// weight matrix for a few dot products, so they are bound by HBM reads of the
// packed weight, not by the matrix cores. Here every weight byte is read
// once, coalesced, dequantized in registers in f32 and used for all M tokens.
//
// A wave covers 16 weight rows: lane t (of 16) walks superblocks t, t+16,
// ..., and each lane serves 4 of the rows with one register copy of the
// activations it needs (a 64-element slice per token at a time); the 16
// partial sums of a row are reduced with lane shuffles. When the
// activations fit in 48 KiB of LDS the variant below is used (activations
// staged in LDS, 64-element units spread over all 16 lanes). Arithmetic is
// f32 throughout, as the reference's batch_matmul_q4k (llm.slang:2264-2365)
// with activations in f32: the register variant forms each weight as
// (d*sc)*q - dmin*mn with one rounding (the FMA below; both products are
// exact), as the reference does; the LDS variant sums the same products as
// d*sc * sum q x - dmin*mn * sum x per 32-element sub-block (the activation
// sums shared by a lane's rows), one FMA per weight instead of two VALU
// operations (double-block modulation launch 379-416 -> 342-371 us).
#include <hip/hip_runtime.h>

#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {
namespace {

template <uint32_t XT>
__device__ __forceinline__ f32x4 load_x4(const void* X, uint64_t e) {
    if constexpr (XT == kGgmlF32) {
        return *(const f32x4*)((const float*)X + e);
    } else {
        const u32x2 v = *(const u32x2*)((const uint16_t*)X + e);
        if constexpr (XT == kGgmlBF16) {
            return f32x4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                         __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
        } else {
            // the halves go through scalars: this compiler's __builtin_bit_cast
            // of a vector element (bit_cast(f16x2, v.y)) reads element 0's bits
            const uint32_t lo = v.x, hi = v.y;
            const f16x2 a = __builtin_bit_cast(f16x2, lo), b = __builtin_bit_cast(f16x2, hi);
            return f32x4{(float)a.x, (float)a.y, (float)b.x, (float)b.y};
        }
    }
}

template <uint32_t XT, int MM>
__global__ void __launch_bounds__(256) gemv_q4k_kernel(const uint8_t* __restrict__ W, const void* __restrict__ X,
                                                        float* __restrict__ Y, uint32_t N, uint32_t K, uint32_t M,
                                                        uint32_t row_offset) {
    // lane t = l % 16 walks superblocks t, t+16, ...; lane group r = l / 16
    // owns rows r, r+4, r+8, r+12 of the wave's 16: one 64-element slice of
    // the activations (per token) is loaded once and used for all four rows
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = lane & 15u, r = lane >> 4;
    const uint32_t n0 = blockIdx.x * 64u + wave * 16u + r;  // rows n0 + 4i, i < 4
    const uint32_t nsb = K / 256u;
    const uint64_t rb = (uint64_t)nsb * 144u;
    float acc[4][MM];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[i][m] = 0.0f;
    for (uint32_t sb = t; sb < nsb; sb += 16u) {
        const uint64_t xb = (uint64_t)sb * 256u;
        u32x4 hdr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t n = n0 + 4u * i;
            hdr[i] = n < N ? *(const u32x4_a4*)(W + (uint64_t)(row_offset + n) * rb + (uint64_t)sb * 144u)
                           : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // activations of elements 64j .. 64j+63 of this superblock, per token
            f32x4 xl[MM][8], xh[MM][8];
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                if (m < (int)M) {
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const uint64_t e = (uint64_t)m * K + xb + 64u * j + 4u * c;
                        xl[m][c] = load_x4<XT>(X, e);
                        xh[m][c] = load_x4<XT>(X, e + 32u);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t n = n0 + 4u * i;
                if (n >= N) continue;
                const uint32_t* b = (const uint32_t*)(W + (uint64_t)(row_offset + n) * rb + (uint64_t)sb * 144u);
                const u32x4 q0 = *(const u32x4_a4*)(b + 4 + 8 * j), q1 = *(const u32x4_a4*)(b + 8 + 8 * j);
                const float d = f16_bits_to_f32(hdr[i].x & 0xffffu), dmin = f16_bits_to_f32(hdr[i].x >> 16);
                uint32_t sc0, mn0, sc1, mn1;
                q4k_scale_min(2u * j, hdr[i].y, hdr[i].z, hdr[i].w, sc0, mn0);
                q4k_scale_min(2u * j + 1u, hdr[i].y, hdr[i].z, hdr[i].w, sc1, mn1);
                const float d0 = d * (float)sc0, m0 = dmin * (float)mn0;
                const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    // bytes 4c .. 4c+3 of the pair's 32 quant bytes: elements
                    // 64j + 4c + k (low nibble) and 64j + 32 + 4c + k (high)
                    const uint32_t word = c < 4 ? q0[c] : q1[c - 4];
                    f32x4 wl, wh;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t q = (word >> (8 * k)) & 0xffu;
                        wl[k] = __builtin_fmaf((float)(q & 15u), d0, -m0);
                        wh[k] = __builtin_fmaf((float)(q >> 4), d1, -m1);
                    }
#pragma unroll
                    for (int m = 0; m < MM; ++m) {
                        if (m < (int)M) {
                            const f32x4 a = xl[m][c], h = xh[m][c];
                            acc[i][m] += (wl.x * a.x + wl.y * a.y) + (wl.z * a.z + wl.w * a.w) +
                                         ((wh.x * h.x + wh.y * h.y) + (wh.z * h.z + wh.w * h.w));
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int m = 0; m < MM; ++m) {
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) acc[i][m] += __shfl_xor(acc[i][m], o, 64);
        }
    if (t == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t n = n0 + 4u * i;
            if (n < N) {
#pragma unroll
                for (int m = 0; m < MM; ++m)
                    if (m < (int)M) Y[(uint64_t)m * N + n] = acc[i][m];
            }
        }
    }
}

// The same products with the activations staged in LDS (f32, once per
// workgroup) and the work of a row split into 64-element units (quarter s
// of superblock sb: its header and 32 quant bytes): lane t of 16 takes units
// t, t+16, ..., so all lanes work whatever K / 256 is, and the next unit's
// weight loads (header and quants of the lane's 4 rows) are issued before
// the current unit is multiplied, keeping two units of loads in flight.
constexpr uint32_t kGemvLdsBytes = 48u * 1024u;

// 4 rows per lane (64 per workgroup): measured against 2 and 1, 4 is as fast
// or faster at every Flux / Z-Image modulation shape.
constexpr int kGemvRowsPerLane = 4;
struct UnitW {
    u32x4 hdr[4], qa[4], qb[4];  // the rows' header and 32 quant bytes of one unit
};

// Up to CAP projections of one shape [N, K] (each its own weight, input
// and output rows, ldy apart): workgroup b serves rows 64 (b % bpj) .. of
// job b / bpj. CAP = 1 for one projection, kGemvMaxJobs for a group.
constexpr uint32_t kGemvMaxJobs = 64;
template <uint32_t CAP>
struct GemvJobs {
    const uint8_t* w[CAP];
    const void* x[CAP];
    float* y[CAP];
    uint32_t m[CAP], row_offset[CAP];
};

template <uint32_t XT, int MM, uint32_t CAP, int RPL = kGemvRowsPerLane>
__global__ void __launch_bounds__(256) gemv_q4k_lds_kernel(const GemvJobs<CAP> jobs, uint32_t N, uint32_t K,
                                                            uint32_t ldy, uint32_t bpj) {
    const uint32_t job = CAP == 1u ? 0u : blockIdx.x / bpj;
    const uint32_t blk = CAP == 1u ? blockIdx.x : blockIdx.x - job * bpj;
    const uint8_t* __restrict__ W = jobs.w[job];
    const void* __restrict__ X = jobs.x[job];
    float* __restrict__ Y = jobs.y[job];
    const uint32_t M = jobs.m[job], row_offset = jobs.row_offset[job];
    extern __shared__ f32x4 xs[];  // [M][K / 4]
    const uint32_t K4 = K / 4u;
#pragma unroll
    for (int m = 0; m < MM; ++m)
        if (m < (int)M)
            for (uint32_t i = threadIdx.x; i < K4; i += 256u) xs[m * K4 + i] = load_x4<XT>(X, (uint64_t)m * K + 4u * i);
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = lane & 15u, r = lane >> 4;
    const uint32_t n0 = blk * (16u * RPL) + wave * (4u * RPL) + r;  // rows n0 + 4i, i < RPL
    const uint32_t U = (K / 256u) * 4u;
    const uint64_t rb = (uint64_t)(K / 256u) * 144u;
    // rows past N read row N - 1 (in bounds, branch-free) and are not stored
    auto load_unit = [&](uint32_t u) __attribute__((always_inline)) {
        const uint32_t sb = u >> 2, j = u & 3u;
        UnitW w;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            const uint32_t n = min(n0 + 4u * i, N - 1u);
            const uint8_t* b = W + (uint64_t)(row_offset + n) * rb + (uint64_t)sb * 144u;
            w.hdr[i] = *(const u32x4_a4*)b;
            w.qa[i] = *(const u32x4_a4*)(b + 16u + 32u * j);
            w.qb[i] = *(const u32x4_a4*)(b + 32u + 32u * j);
        }
        return w;
    };
    float acc[4][MM];
#pragma unroll
    for (int i = 0; i < RPL; i++)
#pragma unroll
        for (int m = 0; m < MM; m++) acc[i][m] = 0.0f;
    // (U >= 4 > t is not guaranteed for K = 256: lanes t >= U have no unit)
    UnitW cur = load_unit(min(t, U - 1u));
    for (uint32_t u = t; u < U; u += 16u) {
        const UnitW nxt = load_unit(min(u + 16u, U - 1u));
        const uint32_t sb = u >> 2, j = u & 3u;
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if (m >= (int)M) continue;
            // activations of elements 64j .. 64j+63 of superblock sb
            const f32x4* xr = xs + m * K4 + sb * 64u + 16u * j;
            f32x4 xl[8], xh[8];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                xl[c] = xr[c];
                xh[c] = xr[c + 8];
            }
            // the sub-blocks' activation sums, shared by the lane's rows
            float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                sxl += (xl[c].x + xl[c].y) + (xl[c].z + xl[c].w);
                sxh += (xh[c].x + xh[c].y) + (xh[c].z + xh[c].w);
            }
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                const float d = f16_bits_to_f32(cur.hdr[i].x & 0xffffu), dmin = f16_bits_to_f32(cur.hdr[i].x >> 16);
                uint32_t sc0, mn0, sc1, mn1;
                q4k_scale_min(2u * j, cur.hdr[i].y, cur.hdr[i].z, cur.hdr[i].w, sc0, mn0);
                q4k_scale_min(2u * j + 1u, cur.hdr[i].y, cur.hdr[i].z, cur.hdr[i].w, sc1, mn1);
                const float d0 = d * (float)sc0, m0 = dmin * (float)mn0;
                const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
                // sum (d0 q - m0) x = d0 sum q x - m0 sum x per 32-element
                // sub-block: one FMA per weight on the nibble as a float
                float ql = 0.0f, qh = 0.0f;
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const uint32_t word = c < 4 ? cur.qa[i][c] : cur.qb[i][c - 4];
                    // nibbles in the bytes of lo / hi; hidden from the compiler's
                    // known bits so each byte converts with one v_cvt_f32_ubyteN
                    // (seen as a 4-bit field it extracts with v_bfe_u32 first)
                    uint32_t lo = word & 0x0f0f0f0fu, hi = (word >> 4) & 0x0f0f0f0fu;
                    asm("" : "+v"(lo), "+v"(hi));
                    const f32x4 a = xl[c], h = xh[c];
                    ql = __builtin_fmaf((float)(lo & 0xffu), a.x, ql);
                    ql = __builtin_fmaf((float)((lo >> 8) & 0xffu), a.y, ql);
                    ql = __builtin_fmaf((float)((lo >> 16) & 0xffu), a.z, ql);
                    ql = __builtin_fmaf((float)(lo >> 24), a.w, ql);
                    qh = __builtin_fmaf((float)(hi & 0xffu), h.x, qh);
                    qh = __builtin_fmaf((float)((hi >> 8) & 0xffu), h.y, qh);
                    qh = __builtin_fmaf((float)((hi >> 16) & 0xffu), h.z, qh);
                    qh = __builtin_fmaf((float)(hi >> 24), h.w, qh);
                }
                acc[i][m] += (d0 * ql - m0 * sxl) + (d1 * qh - m1 * sxh);
            }
        }
        cur = nxt;
    }
#pragma unroll
    for (int i = 0; i < RPL; i++)
#pragma unroll
        for (int m = 0; m < MM; m++) {
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) acc[i][m] += __shfl_xor(acc[i][m], o, 64);
        }
    if (t == 0) {
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const uint32_t n = n0 + 4u * i;
            if (n < N) {
#pragma unroll
                for (int m = 0; m < MM; m++)
                    if (m < (int)M) Y[(uint64_t)m * ldy + n] = acc[i][m];
            }
        }
    }
}

template <uint32_t XT, uint32_t CAP>
void launch_lds(const GemvJobs<CAP>& jobs, uint32_t n_jobs, uint32_t N, uint32_t K, uint32_t ldy, uint32_t max_m,
                hipStream_t st) {
    const uint32_t bpj = (N + 16u * kGemvRowsPerLane - 1u) / (16u * kGemvRowsPerLane);
    const dim3 grid(bpj * n_jobs), block(256);
    const uint32_t lds = max_m * K * 4u;
    if (max_m <= 1)
        hipLaunchKernelGGL((gemv_q4k_lds_kernel<XT, 1, CAP>), grid, block, lds, st, jobs, N, K, ldy, bpj);
    else if (max_m <= 2)
        hipLaunchKernelGGL((gemv_q4k_lds_kernel<XT, 2, CAP>), grid, block, lds, st, jobs, N, K, ldy, bpj);
    else
        hipLaunchKernelGGL((gemv_q4k_lds_kernel<XT, 4, CAP>), grid, block, lds, st, jobs, N, K, ldy, bpj);
}

template <uint32_t XT>
hipError_t launch_t(const void* w, const void* x, float* y, uint32_t N, uint32_t K, uint32_t M, uint32_t row_offset,
                    hipStream_t st) {
    if ((uint64_t)M * K * 4u <= kGemvLdsBytes) {
        const GemvJobs<1> one{{(const uint8_t*)w}, {x}, {y}, {M}, {row_offset}};
        launch_lds<XT>(one, 1u, N, K, N, M, st);
        return hipGetLastError();
    }
    const dim3 grid((N + 63u) / 64u), block(256);
    const uint8_t* W = (const uint8_t*)w;
    if (M <= 1) hipLaunchKernelGGL((gemv_q4k_kernel<XT, 1>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    else if (M <= 2) hipLaunchKernelGGL((gemv_q4k_kernel<XT, 2>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    else hipLaunchKernelGGL((gemv_q4k_kernel<XT, 4>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_q4k_multi(uint32_t xtype, const GemmJob* jobs, uint32_t n_jobs, uint32_t N, uint32_t K,
                                 uint32_t ldy, hipStream_t st) {
    if (n_jobs == 0 || N == 0) return hipSuccess;
    if (n_jobs > kGemvMaxJobs) return hipErrorNotSupported;
    GemvJobs<kGemvMaxJobs> t{};
    uint32_t max_m = 0;
    for (uint32_t q = 0; q < n_jobs; q++) {
        if (jobs[q].M > kGemvMaxTokens || (uint64_t)jobs[q].M * K * 4u > kGemvLdsBytes) return hipErrorNotSupported;
        t.w[q] = (const uint8_t*)jobs[q].w;
        t.x[q] = jobs[q].x;
        t.y[q] = jobs[q].y;
        t.m[q] = jobs[q].M;
        t.row_offset[q] = jobs[q].row_offset;
        max_m = max(max_m, jobs[q].M);
    }
    if (max_m == 0) return hipSuccess;
    switch (xtype) {
        case kGgmlF32: launch_lds<kGgmlF32>(t, n_jobs, N, K, ldy, max_m, st); break;
        case kGgmlF16: launch_lds<kGgmlF16>(t, n_jobs, N, K, ldy, max_m, st); break;
        default: launch_lds<kGgmlBF16>(t, n_jobs, N, K, ldy, max_m, st); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_q4k(const void* w, uint32_t xtype, const void* x, float* y, uint32_t N, uint32_t K,
                           uint32_t M, uint32_t row_offset, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    if (M > kGemvMaxTokens) return hipErrorInvalidValue;
    switch (xtype) {
        case kGgmlF32: return launch_t<kGgmlF32>(w, x, y, N, K, M, row_offset, st);
        case kGgmlF16: return launch_t<kGgmlF16>(w, x, y, N, K, M, row_offset, st);
        default: return launch_t<kGgmlBF16>(w, x, y, N, K, M, row_offset, st);
    }
}

}  // namespace llmr
