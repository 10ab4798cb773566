// synth.hip - synthetic Q4_K weights generated on the device, for workloads
// whose weights do not fit a host-side generator (a full Flux-shaped step has
// ~12 G weights). Same values as llmr_amd.synth.normal followed by
// llmr_amd.gguf.quantize_q4k on the host:
//   element i of stream (seed, stream): counters 2j, 2j+1 (j = i/2) of a
//   SplitMix64 sequence keyed by the stream, Box-Muller in float64, times std,
//   rounded once to f32;
//   each 256-element superblock quantized by the float64 min/max rule (see
//   quantize_q4k), the scales stored as round-to-nearest-even halves.
// One wave per superblock; lane l holds elements 4l .. 4l+3 (sub-block l/8).
#include <hip/hip_runtime.h>

#include "llmr_device.h"
#include "llmr_internal.h"

#pragma clang fp contract(off)

namespace llmr {
namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// float64 -> float16 bits with a single round to nearest even: round to odd
// at f32 (24 >= 11 + 2 bits, so the second rounding cannot double-round),
// then the hardware's RNE f32 -> f16. Inputs here are finite and >= 0.
__device__ __forceinline__ uint16_t f64_to_f16_rne(double x) {
    float f = (float)x;
    if ((double)f != x) {
        uint32_t u = __float_as_uint(f);
        if (fabs((double)f) > fabs(x)) u -= 1u;  // truncate toward zero
        f = __uint_as_float(u | 1u);
    }
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ double f16_bits_to_f64(uint16_t h) {
    return (double)(float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ double shfl_max(double v, int mask) {
    return fmax(v, __shfl_xor(v, mask, 64));
}
__device__ __forceinline__ double shfl_min(double v, int mask) {
    return fmin(v, __shfl_xor(v, mask, 64));
}

__global__ void __launch_bounds__(256) synth_q4k_kernel(uint8_t* __restrict__ out, uint64_t n_sb,
                                                         uint64_t key, double std) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t sb = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6);
    if (sb >= n_sb) return;  // whole wave exits together
    // the four values of this lane: elements e0 .. e0+3 of the stream
    const uint64_t e0 = sb * 256u + 4u * lane;
    double v[4];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const uint64_t j = e0 / 2u + (uint64_t)p;
        const uint64_t b1 = mix64(key + (2u * j + 1u) * kGolden);
        const uint64_t b2 = mix64(key + (2u * j + 2u) * kGolden);
        const double u1 = (double)(b1 >> 11) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(b2 >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log1p(-u1));
        const double th = 2.0 * M_PI * u2;
        v[2 * p] = (double)(float)(r * cos(th) * std);
        v[2 * p + 1] = (double)(float)(r * sin(th) * std);
    }
    // sub-block (8 lanes) min / max, then mn = max(0, -min), sc = (max + mn) / 15
    double lo = fmin(fmin(v[0], v[1]), fmin(v[2], v[3]));
    double hi = fmax(fmax(v[0], v[1]), fmax(v[2], v[3]));
    lo = shfl_min(shfl_min(shfl_min(lo, 1), 2), 4);
    hi = shfl_max(shfl_max(shfl_max(hi, 1), 2), 4);
    const double mn = lo < 0.0 ? -lo : 0.0;
    const double sc = (hi + mn) / 15.0;
    const double dmax = fmax(shfl_max(shfl_max(shfl_max(sc, 8), 16), 32), 0.0);
    const double mmax = fmax(shfl_max(shfl_max(shfl_max(mn, 8), 16), 32), 0.0);
    const uint16_t dbits = f64_to_f16_rne(dmax / 63.0);
    const uint16_t mbits = f64_to_f16_rne(mmax / 63.0);
    const double dd = f16_bits_to_f64(dbits), dm = f16_bits_to_f64(mbits);
    const uint32_t ls = dd > 0.0 ? (uint32_t)fmin(fmax(floor(sc / dd + 0.5), 0.0), 63.0) : 0u;
    const uint32_t lm = dm > 0.0 ? (uint32_t)fmin(fmax(floor(mn / dm + 0.5), 0.0), 63.0) : 0u;
    const double S = dd * (double)ls, O = dm * (double)lm;
    uint32_t q4 = 0;  // the four 4-bit quants, one per byte
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = S > 0.0 ? (uint32_t)fmin(fmax(floor((v[i] + O) / S + 0.5), 0.0), 15.0) : 0u;
        q4 |= q << (8 * i);
    }
    uint8_t* blk = out + sb * 144u;
    // qs[32j + l'] = q[64j + l'] | q[64j + 32 + l'] << 4: lane l (h = (l/8)&1 == 0)
    // pairs with lane l + 8, which holds the same l' in the upper half.
    const uint32_t hi4 = __shfl_xor(q4, 8, 64);
    if (((lane >> 3) & 1u) == 0u) {
        const uint32_t jj = lane >> 4, lp = 4u * (lane & 7u);
        *(uint32_t*)(blk + 16u + 32u * jj + lp) = q4 | (hi4 << 4);
    }
    // the scale field (inverse of get_scale_min_k4) from every sub-block's ls/lm
    uint32_t lsv[8], lmv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        lsv[s] = __shfl(ls, 8 * s, 64);
        lmv[s] = __shfl(lm, 8 * s, 64);
    }
    if (lane == 0) {
        uint8_t s12[12];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s12[j] = (uint8_t)((lsv[j] & 63u) | ((lsv[j + 4] >> 4) << 6));
            s12[j + 4] = (uint8_t)((lmv[j] & 63u) | ((lmv[j + 4] >> 4) << 6));
            s12[j + 8] = (uint8_t)((lsv[j + 4] & 15u) | ((lmv[j + 4] & 15u) << 4));
        }
        u32x4 hdr;
        hdr.x = (uint32_t)dbits | ((uint32_t)mbits << 16);
        hdr.y = s12[0] | (s12[1] << 8) | (s12[2] << 16) | ((uint32_t)s12[3] << 24);
        hdr.z = s12[4] | (s12[5] << 8) | (s12[6] << 16) | ((uint32_t)s12[7] << 24);
        hdr.w = s12[8] | (s12[9] << 8) | (s12[10] << 16) | ((uint32_t)s12[11] << 24);
        *(u32x4*)blk = hdr;
    }
}

uint64_t stream_key(uint64_t seed, uint64_t stream) {
    const uint64_t z = seed * 0x100000001B3ull + stream * 0x632BE59BD9B4E019ull;  // mod 2^64
    uint64_t x = z;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

}  // namespace

hipError_t launch_synth_q4k(void* out, uint64_t n_rows, uint32_t in_dim, uint64_t seed, uint64_t stream,
                            double std, hipStream_t st) {
    const uint64_t n_sb = n_rows * (in_dim / 256u);
    if (n_sb == 0) return hipSuccess;
    const uint64_t grid = (n_sb + 3u) / 4u;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(synth_q4k_kernel, dim3((uint32_t)grid), dim3(256), 0, st, (uint8_t*)out, n_sb,
                       stream_key(seed, stream), std);
    return hipGetLastError();
}

}  // namespace llmr
