// dequant.hip - GGUF Q8_0 / Q4_K dequantization kernels (the bit-exactness
// contract of the backend) for gfx950.
//
// f32 form: bit-exact to dequant_q8_0_block (lib/model/tensor.c3:354-361) and
// dequant_q4k_block (lib/model/tensor.c3:292-335).
// fp16 operand form: exactly the values the GEMM feeds the matrix cores; the
// Q8_0 conversion is the same device function the GEMM's weight loader uses.
//
// HBM-bound byte work: one thread per 8 consecutive outputs of a row, reading
// the packed block bytes it needs and writing 32 B (f32) or 16 B (fp16).
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Eight consecutive Q8_0 quants (bytes) starting at p, as two little-endian dwords.
__device__ __forceinline__ void ld_q8x8(const uint8_t* p, uint32_t& w0, uint32_t& w1) {
    w0 = ld_u8(p) | (ld_u8(p + 1) << 8) | (ld_u8(p + 2) << 16) | (ld_u8(p + 3) << 24);
    w1 = ld_u8(p + 4) | (ld_u8(p + 5) << 8) | (ld_u8(p + 6) << 16) | (ld_u8(p + 7) << 24);
}

// Q4_K: value of element e (0..255) of the superblock at blk, f32,
// d*sc*q - dmin*mn with d*sc and d*sc*q exact (llm.slang:2321-2328).
__device__ __forceinline__ float q4k_value(const uint8_t* blk, uint32_t e, float d, float dmin,
                                           uint32_t s0, uint32_t s1, uint32_t s2) {
    const uint32_t j = e >> 6, h = (e >> 5) & 1u, l = e & 31u;
    uint32_t sc, mn;
    q4k_scale_min(2 * j + h, s0, s1, s2, sc, mn);
    const uint32_t qb = ld_u8(blk + 16 + j * 32 + l);
    const uint32_t q = h ? (qb >> 4) : (qb & 0xfu);
    const float dsc = d * (float)sc;
    const float dmn = dmin * (float)mn;
    return dsc * (float)q - dmn;
}

template <bool kOperand>
__global__ void __launch_bounds__(256) dequant_q8_0_kernel(const uint8_t* __restrict__ w,
                                                           uint32_t n_rows, uint32_t in_dim,
                                                           uint32_t row_offset, void* __restrict__ out) {
    const uint32_t groups_per_row = in_dim / 8;
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)n_rows * groups_per_row) return;
    const uint32_t r = (uint32_t)(gid / groups_per_row);
    const uint32_t g = (uint32_t)(gid % groups_per_row);
    const uint32_t k0 = g * 8;
    const uint64_t row_bytes = (uint64_t)(in_dim / 32) * 34;
    const uint8_t* blk = w + (uint64_t)(row_offset + r) * row_bytes + (uint64_t)(k0 / 32) * 34;
    const uint32_t dbits = ld_u16(blk);
    uint32_t w0, w1;
    ld_q8x8(blk + 2 + (k0 % 32), w0, w1);
    const uint64_t o = (uint64_t)r * in_dim + k0;
    if (kOperand) {
        const _Float16 dh = (_Float16)f16_bits_to_f32(dbits);
        const f16x2 d2 = {dh, dh};
        const f16x4 a = q8x4_to_f16(w0, d2);
        const f16x4 b = q8x4_to_f16(w1, d2);
        f16x8 v;
        v.s0 = a.x; v.s1 = a.y; v.s2 = a.z; v.s3 = a.w;
        v.s4 = b.x; v.s5 = b.y; v.s6 = b.z; v.s7 = b.w;
        *(f16x8*)((uint16_t*)out + o) = v;
    } else {
        const float d = f16_bits_to_f32(dbits);
        f32x4 a, b;
        a.x = d * (float)(int8_t)(w0 & 0xffu);
        a.y = d * (float)(int8_t)((w0 >> 8) & 0xffu);
        a.z = d * (float)(int8_t)((w0 >> 16) & 0xffu);
        a.w = d * (float)(int8_t)(w0 >> 24);
        b.x = d * (float)(int8_t)(w1 & 0xffu);
        b.y = d * (float)(int8_t)((w1 >> 8) & 0xffu);
        b.z = d * (float)(int8_t)((w1 >> 16) & 0xffu);
        b.w = d * (float)(int8_t)(w1 >> 24);
        float* of = (float*)out + o;
        *(f32x4*)of = a;
        *(f32x4*)(of + 4) = b;
    }
}

template <bool kOperand>
__global__ void __launch_bounds__(256) dequant_q4k_kernel(const uint8_t* __restrict__ w,
                                                          uint32_t n_rows, uint32_t in_dim,
                                                          uint32_t row_offset, void* __restrict__ out) {
    const uint32_t groups_per_row = in_dim / 8;
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)n_rows * groups_per_row) return;
    const uint32_t r = (uint32_t)(gid / groups_per_row);
    const uint32_t g = (uint32_t)(gid % groups_per_row);
    const uint32_t k0 = g * 8;
    const uint64_t row_bytes = (uint64_t)(in_dim / 256) * 144;
    const uint8_t* blk = w + (uint64_t)(row_offset + r) * row_bytes + (uint64_t)(k0 / 256) * 144;
    const float d = f16_bits_to_f32(ld_u16(blk));
    const float dmin = f16_bits_to_f32(ld_u16(blk + 2));
    const uint32_t s0 = *(const uint32_t*)(blk + 4);
    const uint32_t s1 = *(const uint32_t*)(blk + 8);
    const uint32_t s2 = *(const uint32_t*)(blk + 12);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = q4k_value(blk, (k0 % 256) + i, d, dmin, s0, s1, s2);
    const uint64_t o = (uint64_t)r * in_dim + k0;
    if (kOperand) {
        u32x4 p;
        p.x = pack_f16x2(v[0], v[1]);
        p.y = pack_f16x2(v[2], v[3]);
        p.z = pack_f16x2(v[4], v[5]);
        p.w = pack_f16x2(v[6], v[7]);
        *(u32x4*)((uint16_t*)out + o) = p;
    } else {
        float* of = (float*)out + o;
        *(f32x4*)of = f32x4{v[0], v[1], v[2], v[3]};
        *(f32x4*)(of + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
}

}  // namespace

static hipError_t launch_dequant(const void* w, uint32_t wtype, uint32_t n_rows, uint32_t in_dim,
                                 uint32_t row_offset, void* out, bool operand, hipStream_t st) {
    const uint64_t threads = (uint64_t)n_rows * (in_dim / 8);
    if (threads == 0) return hipSuccess;
    const uint32_t blocks = (uint32_t)((threads + 255) / 256);
    const uint8_t* wp = (const uint8_t*)w;
    if (wtype == kGgmlQ8_0) {
        if (operand)
            dequant_q8_0_kernel<true><<<blocks, 256, 0, st>>>(wp, n_rows, in_dim, row_offset, out);
        else
            dequant_q8_0_kernel<false><<<blocks, 256, 0, st>>>(wp, n_rows, in_dim, row_offset, out);
    } else {
        if (operand)
            dequant_q4k_kernel<true><<<blocks, 256, 0, st>>>(wp, n_rows, in_dim, row_offset, out);
        else
            dequant_q4k_kernel<false><<<blocks, 256, 0, st>>>(wp, n_rows, in_dim, row_offset, out);
    }
    return hipGetLastError();
}

hipError_t launch_dequant_f32(const void* w, uint32_t wtype, uint32_t n_rows, uint32_t in_dim,
                              uint32_t row_offset, float* out, hipStream_t st) {
    return launch_dequant(w, wtype, n_rows, in_dim, row_offset, out, false, st);
}

hipError_t launch_dequant_operand_f16(const void* w, uint32_t wtype, uint32_t n_rows,
                                      uint32_t in_dim, uint32_t row_offset, uint16_t* out,
                                      hipStream_t st) {
    return launch_dequant(w, wtype, n_rows, in_dim, row_offset, out, true, st);
}

}  // namespace llmr
