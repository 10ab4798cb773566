// gemv_q.hip - Q4_K dequant-GEMM for a handful of tokens (M <= 8): the
// modulation and timestep projections of a DiT step (M = 1) stream a whole
// weight matrix for a few dot products, so they are bound by HBM reads of the
// packed weight, not by the matrix cores. Here every weight byte is read
// once, coalesced, dequantized in registers in f32 and used for all M tokens.
//
// Sixteen lanes per weight row: lane t of a row walks superblocks t, t+16, ...
// (144 contiguous bytes each), a wave covers 4 rows and a workgroup 16; the
// 16 partial sums of a row are reduced with lane shuffles. Arithmetic is the
// reference's f32 path (batch_matmul_q4k, llm.slang:2264-2365): weight
// (d*sc)*q - dmin*mn with one rounding (the FMA below; both products are
// exact), activations in f32, f32 accumulation (in a different order).
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
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t = lane & 15u;
    const uint32_t n = blockIdx.x * 16u + wave * 4u + (lane >> 4);
    const uint32_t nsb = K / 256u;
    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
    if (n < N) {
        const uint8_t* wr = W + (uint64_t)(row_offset + n) * nsb * 144u;
        for (uint32_t sb = t; sb < nsb; sb += 16u) {
            const uint32_t* b = (const uint32_t*)(wr + (uint64_t)sb * 144u);  // dword-aligned
            const u32x4 hdr = *(const u32x4_a4*)b;
            u32x4 qs[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) qs[i] = *(const u32x4_a4*)(b + 4 + 4 * i);
            const float d = f16_bits_to_f32(hdr.x & 0xffffu), dmin = f16_bits_to_f32(hdr.x >> 16);
            const uint64_t xb = (uint64_t)sb * 256u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t sc0, mn0, sc1, mn1;
                q4k_scale_min(2u * j, hdr.y, hdr.z, hdr.w, sc0, mn0);
                q4k_scale_min(2u * j + 1u, hdr.y, hdr.z, hdr.w, sc1, mn1);
                const float d0 = d * (float)sc0, m0 = dmin * (float)mn0;
                const float d1 = d * (float)sc1, m1 = dmin * (float)mn1;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    // bytes 4c .. 4c+3 of the pair's 32 quant bytes: elements
                    // 64j + 4c + i (low nibble) and 64j + 32 + 4c + i (high)
                    const uint32_t word = qs[2 * j + c / 4][c % 4];
                    f32x4 wl, wh;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t q = (word >> (8 * i)) & 0xffu;
                        wl[i] = __builtin_fmaf((float)(q & 15u), d0, -m0);
                        wh[i] = __builtin_fmaf((float)(q >> 4), d1, -m1);
                    }
#pragma unroll
                    for (int m = 0; m < MM; ++m) {
                        if (m < (int)M) {
                            const uint64_t e = (uint64_t)m * K + xb + 64u * j + 4u * c;
                            const f32x4 xl = load_x4<XT>(X, e), xh = load_x4<XT>(X, e + 32u);
                            acc[m] += (wl.x * xl.x + wl.y * xl.y) + (wl.z * xl.z + wl.w * xl.w) +
                                      ((wh.x * xh.x + wh.y * xh.y) + (wh.z * xh.z + wh.w * xh.w));
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o, 64);
    }
    if (t == 0 && n < N) {
#pragma unroll
        for (int m = 0; m < MM; ++m)
            if (m < (int)M) Y[(uint64_t)m * N + n] = acc[m];
    }
}

template <uint32_t XT>
hipError_t launch_t(const void* w, const void* x, float* y, uint32_t N, uint32_t K, uint32_t M, uint32_t row_offset,
                    hipStream_t st) {
    const dim3 grid((N + 15u) / 16u), block(256);
    const uint8_t* W = (const uint8_t*)w;
    if (M <= 1) hipLaunchKernelGGL((gemv_q4k_kernel<XT, 1>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    else if (M <= 2) hipLaunchKernelGGL((gemv_q4k_kernel<XT, 2>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    else if (M <= 4) hipLaunchKernelGGL((gemv_q4k_kernel<XT, 4>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    else hipLaunchKernelGGL((gemv_q4k_kernel<XT, 8>), grid, block, 0, st, W, x, y, N, K, M, row_offset);
    return hipGetLastError();
}

}  // namespace

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
