// llmr_device.h - device-side types and helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace llmr {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 16-byte vector that is only guaranteed 4-byte aligned (GGUF Q8_0 rows are
// dword-aligned but not 16-byte aligned); global_load_dwordx4 needs dword alignment.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr uint32_t kGgmlF32 = 0, kGgmlF16 = 1, kGgmlQ8_0 = 8, kGgmlQ4K = 12, kGgmlBF16 = 30;

// f(std::integral_constant<int, I>) for I = B .. E-1, unrolled at compile time
// (every index derived from I is a constant expression).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Buffer resource over [base, base + bytes): loads past the end return zero
// and stores past it are dropped (raw buffer, dword format word 3).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint64_t bytes) {
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// s_waitcnt vmcnt(n) leaving the LDS and export counters unconstrained
// (gfx9 encoding: vmcnt[3:0] | expcnt << 4 | lgkmcnt << 8 | vmcnt[5:4] << 14).
#define LLMR_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

// Workgroup barrier for a pipelined loop: this wave's LDS accesses are done
// (lgkmcnt(0)) and at most `n` of its global loads/DMAs are still in flight,
// then s_barrier. __syncthreads() would instead wait for every outstanding
// global load (vmcnt(0)), i.e. for the prefetches issued for later stages.
// The empty asm statements keep the compiler from moving memory operations
// across the barrier.
#define LLMR_STAGE_BARRIER(n)                                                              \
    do {                                                                                   \
        asm volatile("" ::: "memory");                                                     \
        __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (0 << 8) | (((n) >> 4) << 14)); \
        __builtin_amdgcn_s_barrier();                                                      \
        asm volatile("" ::: "memory");                                                     \
    } while (0)

// fp16 bit pattern -> f32 exactly as unpack_f16 (llm.slang:235-251) and
// cpu_f16_to_f32 (tensor.c3:130-147): exponent 31 (Inf and every NaN) -> +-Inf;
// everything else is the exact value (the hardware widening is exact for
// zero, subnormal and normal halves).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
    const float inf = __uint_as_float(((bits & 0x8000u) << 16) | 0x7f800000u);
    return ((bits & 0x7c00u) == 0x7c00u) ? inf : v;
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    f16x2 h;
    h.x = (_Float16)a;  // round to nearest even (v_cvt_pk_f16_f32)
    h.y = (_Float16)b;
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)a, (__bf16)b});  // nearest even (v_cvt_pk_bf16_f32)
}

// Two bf16 halves of a dword -> their f16 roundings, packed.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
    return pack_f16x2(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

// Eight int8 values (two dwords) times an fp16 scale -> eight fp16 RN16(d*q),
// the Q8_0 matrix operand of batch_matmul_q8 (llm.slang:1699-1703:
// float16_t s * float16_t(q)). int8 -> fp16 is exact via the 1024+128+q bias
// trick, the product is one IEEE fp16 multiply (round to nearest even).
__device__ __forceinline__ f16x4 q8x4_to_f16(uint32_t w, f16x2 d2) {
    const uint32_t x = w ^ 0x80808080u;                       // q + 128 in each byte
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);  // 0x64|b1, 0x64|b0
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);  // 0x64|b3, 0x64|b2
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    f16x2 a = __builtin_bit_cast(f16x2, lo) - bias;  // exact q0, q1
    f16x2 b = __builtin_bit_cast(f16x2, hi) - bias;  // exact q2, q3
    a = a * d2;
    b = b * d2;
    f16x4 r;
    r.x = a.x; r.y = a.y; r.z = b.x; r.w = b.y;
    return r;
}

// Two 4-bit quants (bytes of `nib` picked by the v_perm selector `sel`, each
// 0..15) -> packed fp16 RN16(dsc*q - dmn): 0x6400|q is the half 1024+q, one
// packed subtract gives q exactly, and the mixed-precision FMA
// (v_fma_mix{lo,hi}_f16) rounds the exact dsc*q - dmn once.
__device__ __forceinline__ uint32_t q4_pair(uint32_t nib, uint32_t sel, float dsc, float dmn) {
    const f16x2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    const f16x2 q = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, nib, sel)) - bias;
    f16x2 r;
    r.x = (_Float16)__builtin_fmaf((float)q.x, dsc, -dmn);
    r.y = (_Float16)__builtin_fmaf((float)q.y, dsc, -dmn);
    return __builtin_bit_cast(uint32_t, r);
}

// The same two quants as packed bf16: the reference's f32 value d*sc*q - dmin*mn
// (both products exact, one rounding in the FMA) rounded to bf16.
__device__ __forceinline__ uint32_t q4_pair_bf16(uint32_t nib, uint32_t sel, float dsc, float dmn) {
    const uint32_t q = __builtin_amdgcn_perm(0u, nib, sel);  // q0 in bits 0-7, q1 in bits 16-23
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t r;
    r.x = (__bf16)__builtin_fmaf((float)(q & 0xffu), dsc, -dmn);
    r.y = (__bf16)__builtin_fmaf((float)(q >> 16), dsc, -dmn);
    return __builtin_bit_cast(uint32_t, r);
}

// get_scale_min_k4 (llm.slang:447-462) for sub-block index `is` (wave-uniform)
// on the 12 scale bytes held in dwords s0 (bytes 0-3), s1 (4-7), s2 (8-11).
// Branch-free (a mask select) so a loop calling it stays one basic block.
__device__ __forceinline__ void q4k_scale_min(uint32_t is, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t& sc, uint32_t& mn) {
    const uint32_t sh = 8u * (is & 3u);
    const uint32_t x0 = (s0 >> sh) & 0xffu;  // byte is (is < 4) or byte is-4 (is >= 4)
    const uint32_t x1 = (s1 >> sh) & 0xffu;  // byte is+4 (is < 4) or byte is (is >= 4)
    const uint32_t x2 = (s2 >> sh) & 0xffu;  // byte is+4 (is >= 4)
    const uint32_t hi = 0u - (is >> 2);      // all ones when is >= 4
    sc = ((x0 & 63u) & ~hi) | (((x2 & 0xfu) | ((x0 >> 6) << 4)) & hi);
    mn = ((x1 & 63u) & ~hi) | (((x2 >> 4) | ((x1 >> 6) << 4)) & hi);
}

}  // namespace llmr
