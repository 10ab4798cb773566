// gemm_q_common.h - pieces shared by the persistent dequant-GEMM kernels
// (gemm_q.hip) and the two-pass GEMM (gemm_w16.hip): the LDS tile layout,
// the 32x32x16 MFMA on 16-bit operands, the per-row weight dequantization
// of one 64-wide K stage, the tile order and the epilogue arguments.
#pragma once

#include <type_traits>

#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

// One GEMM of a persistent launch. A launch multiplies up to two problems
// that share N and K (e.g. the text and image rows of a block with their own
// weights); their 256-row tiles are stacked along M, problem 0 first.
struct PersistProblem {
    const uint8_t* W;   // weight blocks; row row_offset is output feature 0
    const void* X;      // [M, K] 16-bit activations
    float* Y;           // f32 output (kEpiResidual: read and updated)
    const float* gate;  // kEpiResidual: [N] or null
    void* Y2;           // kEpiSplitGelu: 16-bit output
    uint32_t M, row_offset, tiles_m;
};
// Weight images of later GEMM groups, built by the two-pass GEMM's
// workgroups that have no tile in its last round (items: (panel, group of 4
// stages) of w16_image_kernel, numbered across the images in order, image
// i's item u at first[i] + u; the first `items` of them here, the rest by
// w16_image_kernel after the GEMM).
struct NextImages {
    const uint8_t* W[8];   // raw weight blocks, row row_offset[i] is feature 0
    const uint8_t* W2[8];  // non-null: a SwiGLU-arranged image, W[i] its gate rows, W2[i] its up rows
    uint8_t* img[8];
    uint32_t row_offset[8], N[8], K[8], first[8];
    uint32_t count, wtype;
    uint32_t items;       // items built by the GEMM's idle workgroups (0: none)
};
// Head routing of the split-epilogue GEMMs' first `split` = 3 H 128 output
// features (q non-null): feature slot * H * 128 + head * 128 + f (slot Q, K,
// V) of token m of problem p goes, per-head RMS-normalised (Q, K with a norm
// weight) and rotated (Q, K with tables), to dst_slot[head, row0[p] + m, f]
// in 16 bits instead of to Y.
struct HeadsEpi {
    void* q;  // [n_heads, seq, 128] each; null: no head routing
    void* k;
    void* v;
    const float* cos;  // [seq, 64] or null
    const float* sin;
    const float* qn[2];  // per problem: [128] or null
    const float* kn[2];
    uint32_t row0[2];
    uint32_t n_heads, seq, out_bf16;
    float eps;
};
struct PersistArgs {
    PersistProblem p[2];
    const uint8_t* W2;  // SwiGLU: the up weight (p[0].W is the gate)
    uint32_t N, K, tiles_m, tiles_n;  // tiles_m of both problems
    uint32_t epi, ldy, ldy2, split, y2_bf16;
    HeadsEpi heads;
    NextImages next;
};

// The persistent all-DMA GEMM over weight images (gemm_w16.hip): p[i].W is
// the image of problem i (launch_w16_image); swiglu: one 128-feature SwiGLU
// image; grouped: two problems.
hipError_t launch_w16_gemm(const PersistArgs& a, uint32_t xtype, bool swiglu, bool grouped, int num_cus,
                           hipStream_t st);

namespace {

constexpr int kBK = 64;  // K per stage

// Bank swizzle of 128-byte LDS rows (eight 16-byte chunks): chunk c of row r
// sits at physical chunk c ^ lds_swz(r). A 16-byte fragment read touches one
// chunk of consecutive rows; lds_swz gives any 8 consecutive rows (one
// 128-byte bank line each) 8 distinct chunk positions, and the 8 even and the
// 8 odd rows of any 16 consecutive ones (two rows per 256-byte line of the
// 64 banks) 8 distinct positions each, so the read is conflict-free whether
// the hardware serves 8 or 16 lanes of a 16-byte access per cycle.
__device__ __forceinline__ uint32_t lds_swz(uint32_t r) { return (r & 7u) ^ ((r >> 3) & 1u); }
__device__ __forceinline__ uint32_t lds_off(uint32_t r, uint32_t c) {
    return r * 128u + ((c ^ lds_swz(r)) << 4);
}

// 32x32x16 MFMA on 16-bit operand bits: bf16 operands for bf16 activations
// (fp16 cannot hold bf16's range), fp16 otherwise.
template <uint32_t XT>
__device__ __forceinline__ f32x16 mfma16(f16x8 a, f16x8 b, f32x16 c) {
    if constexpr (XT == kGgmlBF16) {
        typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
}

__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
// Eight Q8_0 quants (two dwords) -> one 16-byte chunk of fp16 operands RN16(d*q).
__device__ __forceinline__ u32x4 q8x8_f16(uint32_t q0, uint32_t q1, f16x2 d2) {
    const f16x4 lo = q8x4_to_f16(q0, d2), hi = q8x4_to_f16(q1, d2);
    return __builtin_bit_cast(u32x4, f16x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
}

// Tile order: in every full round of G = gridDim.x tiles the 32 workgroups
// one XCD runs (dispatch is round-robin over the 8 XCDs) get 32 consecutive
// indices, which the group-of-4-tile-rows order turns into a 4 x 8 block of
// tiles (4 x 256 activation rows and 8 x 256 weight rows shared in the XCD's L2).
__device__ __forceinline__ void tile_of_linear(uint32_t L, uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm,
                                               uint32_t& tn);
__device__ __forceinline__ void map_tile_persist(uint32_t T, uint32_t G, uint32_t tiles_m, uint32_t tiles_n,
                                                 uint32_t& tm, uint32_t& tn) {
    constexpr uint32_t kXcd = 8;
    const uint32_t total = tiles_m * tiles_n;
    uint32_t L = T;
    if (G % kXcd == 0 && T / G < total / G) {
        const uint32_t b = T % G;
        L = (T - b) + (b % kXcd) * (G / kXcd) + b / kXcd;
    }
    tile_of_linear(L, tiles_m, tiles_n, tm, tn);
}

// The two-pass kernel's order (grid G = the CUs, G % 8 == 0): full rounds as
// map_tile_persist; the last, part-filled round of rem = total % G tiles is
// split into 8 contiguous runs of rem / 8 (+1 for the first rem % 8 XCDs),
// one per XCD, taken by that XCD's first workgroups (j = b / 8), so each
// XCD's L2 serves neighbouring tiles and every XCD keeps the same number of
// idle workgroups. Workgroup b's tile count, its k-th tile, and its rank
// among the workgroups without a tile in the last round (rem > 0).
__device__ __forceinline__ uint32_t w16_n_tiles(uint32_t b, uint32_t G, uint32_t total) {
    const uint32_t R = total / G, rem = total % G;
    if (G % 8u) return R + (b < rem ? 1u : 0u);
    const uint32_t x = b % 8u, j = b / 8u;
    return R + (j < rem / 8u + (x < rem % 8u ? 1u : 0u) ? 1u : 0u);
}
__device__ __forceinline__ void w16_tile(uint32_t b, uint32_t k, uint32_t G, uint32_t tiles_m, uint32_t tiles_n,
                                         uint32_t& tm, uint32_t& tn) {
    const uint32_t total = tiles_m * tiles_n, R = total / G, rem = total % G;
    uint32_t L = k * G + b;
    if (G % 8u == 0) {
        const uint32_t x = b % 8u, j = b / 8u;
        L = k < R ? k * G + x * (G / 8u) + j : R * G + x * (rem / 8u) + min(x, rem % 8u) + j;
    }
    tile_of_linear(L, tiles_m, tiles_n, tm, tn);
}
__device__ __forceinline__ uint32_t w16_idle_rank(uint32_t b, uint32_t G, uint32_t total) {
    const uint32_t rem = total % G;
    if (G % 8u) return b - rem;
    const uint32_t x = b % 8u, j = b / 8u, q = rem / 8u, e = rem % 8u;
    return x * (G / 8u) - x * q - min(x, e) + j - (q + (x < e ? 1u : 0u));
}

// Linear tile index -> (tile row, tile column) in groups of 4 tile rows.
__device__ __forceinline__ void tile_of_linear(uint32_t L, uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm,
                                               uint32_t& tn) {
    constexpr uint32_t kGroupM = 4;
    const uint32_t per_group = kGroupM * tiles_n;
    const uint32_t g = L / per_group;
    const uint32_t first_m = g * kGroupM;
    const uint32_t gsize = min(tiles_m - first_m, kGroupM);
    const uint32_t in = L % per_group;
    tm = first_m + in % gsize;
    tn = in / gsize;
}

// Bytes 0,1 (SEL_LO) or 2,3 (SEL_HI) of `w` as two fp16 subnormals b * 2^-24
// (exact: the byte is the mantissa of a zero-exponent half), so one mixed
// FMA with a scale pre-multiplied by 2^24 forms scale * b + bias exactly
// before its single rounding - no bias subtraction of the 1024+b encoding.
constexpr uint32_t kSelLo = 0x0c010c00u, kSelHi = 0x0c030c02u;
__device__ __forceinline__ f16x2 sub16x2(uint32_t w, uint32_t sel) {
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, w, sel));
}
// Two operands RN(s * h + b) of type OT from the two halves of h, packed.
template <uint32_t OT>
__device__ __forceinline__ uint32_t fma_pair(f16x2 h, float s, float b) {
    if constexpr (OT == kGgmlBF16) {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        bf16x2_t r;
        r.x = (__bf16)__builtin_fmaf((float)h.x, s, b);
        r.y = (__bf16)__builtin_fmaf((float)h.y, s, b);
        return __builtin_bit_cast(uint32_t, r);
    } else {
        f16x2 r;
        r.x = (_Float16)__builtin_fmaf((float)h.x, s, b);
        r.y = (_Float16)__builtin_fmaf((float)h.y, s, b);
        return __builtin_bit_cast(uint32_t, r);
    }
}

template <uint32_t WT, uint32_t OT>
struct WRow;

// Q4_K row stage s: quarter s % 4 of superblock s / 4 = the 16-byte header
// and qs bytes [32 (s%4), +32): low nibbles are k 0..31 of the stage
// (sub-block 2j), high nibbles k 32..63 (sub-block 2j+1).
// The dequantization is split in four parts (one per 16-wide k step of the
// stage it overlaps): part p writes LDS chunks p and 4+p of the row.
template <uint32_t OT>
struct WRow<kGgmlQ4K, OT> {
    static constexpr int kLoads = 3;
    u32x4 hdr, qa, qb;
    template <int L>
    __device__ __forceinline__ void load(rsrc_t r, uint32_t voff, uint32_t s) {
        const uint32_t sh = (s >> 2) * 144u;
        const uint32_t sq = sh + 16u + 32u * (s & 3u);
        if constexpr (L == 0) hdr = bload16(r, voff, sh);
        if constexpr (L == 1) qa = bload16(r, voff, sq);
        if constexpr (L == 2) qb = bload16(r, voff + 16u, sq);
    }
    // Operand = RN(d*sc*q - dmin*mn) (products exact, one rounding): low
    // nibbles are read as q * 2^-24, high nibbles (masked in place) as
    // 16 q * 2^-24, so their scales carry 2^24 and 2^20.
    struct Scale {
        float s0, b0, s1, b1;
    };
    __device__ __forceinline__ Scale scale(uint32_t s) const {
        const uint32_t j = s & 3u;
        const float d = f16_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(hdr.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(2 * j, hdr.y, hdr.z, hdr.w, sc0, mn0);
        q4k_scale_min(2 * j + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
        return Scale{d * (float)sc0 * 16777216.0f, -(dmin * (float)mn0), d * (float)sc1 * 1048576.0f,
                     -(dmin * (float)mn1)};
    }
    // `base` = LDS offset of chunk 0 of the row; chunk c is at base ^ (c << 4)
    template <int P>
    __device__ __forceinline__ void store(uint8_t* lds, const Scale& c, uint32_t base) const {
        const uint32_t w0 = P < 2 ? qa[2 * P] : qb[2 * P - 4];
        const uint32_t w1 = P < 2 ? qa[2 * P + 1] : qb[2 * P - 3];
        const uint32_t l0 = w0 & 0x0f0f0f0fu, l1 = w1 & 0x0f0f0f0fu;
        const uint32_t h0 = w0 & 0xf0f0f0f0u, h1 = w1 & 0xf0f0f0f0u;
        const u32x4 lo = {fma_pair<OT>(sub16x2(l0, kSelLo), c.s0, c.b0), fma_pair<OT>(sub16x2(l0, kSelHi), c.s0, c.b0),
                          fma_pair<OT>(sub16x2(l1, kSelLo), c.s0, c.b0), fma_pair<OT>(sub16x2(l1, kSelHi), c.s0, c.b0)};
        const u32x4 hi = {fma_pair<OT>(sub16x2(h0, kSelLo), c.s1, c.b1), fma_pair<OT>(sub16x2(h0, kSelHi), c.s1, c.b1),
                          fma_pair<OT>(sub16x2(h1, kSelLo), c.s1, c.b1), fma_pair<OT>(sub16x2(h1, kSelHi), c.s1, c.b1)};
        *(u32x4*)(lds + (base ^ ((uint32_t)P << 4))) = lo;
        *(u32x4*)(lds + (base ^ ((uint32_t)(4 + P) << 4))) = hi;
    }
};

// Q8_0 row stage s: blocks 2s and 2s+1 = bytes [68 s, 68 s + 68) of the row
// (dword-aligned: K % 64 == 0). Block 0: scale in the low half of dword 0,
// quants from byte 2 (chunks 0..3); block 1: scale in the high half of dword
// 8, quants in dwords 9..16 (chunks 4..7). Part p writes chunks p and 4+p.
template <uint32_t OT>
struct WRow<kGgmlQ8_0, OT> {
    static constexpr int kLoads = 5;
    u32x4 a, b, c, d;
    uint32_t e;
    template <int L>
    __device__ __forceinline__ void load(rsrc_t r, uint32_t voff, uint32_t s) {
        const uint32_t so = 68u * s;
        if constexpr (L == 0) a = bload16(r, voff, so);
        if constexpr (L == 1) b = bload16(r, voff + 16u, so);
        if constexpr (L == 2) c = bload16(r, voff + 32u, so);
        if constexpr (L == 3) d = bload16(r, voff + 48u, so);
        if constexpr (L == 4) e = bload4(r, voff + 64u, so);
    }
    struct Scale {
        float s0, b0, s1, b1;  // bf16: (2^24 d, -128 d) per block; f16: (d, -) per block
    };
    __device__ __forceinline__ Scale scale(uint32_t s) const {
        (void)s;
        const float d0 = f16_bits_to_f32(a.x & 0xffffu);
        const float d1 = f16_bits_to_f32(c.x >> 16);
        if constexpr (OT == kGgmlBF16)
            return Scale{d0 * 16777216.0f, -128.0f * d0, d1 * 16777216.0f, -128.0f * d1};
        else
            return Scale{d0, 0.0f, d1, 0.0f};
    }
    __device__ __forceinline__ uint32_t word(int i) const {
        return i < 4 ? a[i] : i < 8 ? b[i - 4] : i < 12 ? c[i - 8] : i < 16 ? d[i - 12] : e;
    }
    // chunk ch of the stage from its two quant dwords q0, q1
    __device__ __forceinline__ u32x4 chunk(uint32_t q0, uint32_t q1, float sc, float bi) const {
        if constexpr (OT == kGgmlBF16) {
            // RN_bf16(d*q): q + 128 read as a subnormal half, d*q = (2^24 d) h - 128 d
            // exactly in f32, then one rounding to bf16
            const uint32_t u0 = q0 ^ 0x80808080u, u1 = q1 ^ 0x80808080u;
            return u32x4{fma_pair<OT>(sub16x2(u0, kSelLo), sc, bi), fma_pair<OT>(sub16x2(u0, kSelHi), sc, bi),
                         fma_pair<OT>(sub16x2(u1, kSelLo), sc, bi), fma_pair<OT>(sub16x2(u1, kSelHi), sc, bi)};
        } else {
            const _Float16 h = (_Float16)sc;
            return q8x8_f16(q0, q1, f16x2{h, h});
        }
    }
    template <int P>
    __device__ __forceinline__ void store(uint8_t* lds, const Scale& k, uint32_t base) const {
        const uint32_t q0 = __builtin_amdgcn_alignbyte(word(2 * P + 1), word(2 * P), 2);
        const uint32_t q1 = __builtin_amdgcn_alignbyte(word(2 * P + 2), word(2 * P + 1), 2);
        *(u32x4*)(lds + (base ^ ((uint32_t)P << 4))) = chunk(q0, q1, k.s0, k.b0);
        *(u32x4*)(lds + (base ^ ((uint32_t)(4 + P) << 4))) = chunk(word(9 + 2 * P), word(10 + 2 * P), k.s1, k.b1);
    }
};


// Schedule of one 16-wide k step inside a stage: its 16 MFMAs each followed
// by a share of the stage's other work, so that work issues while the
// matrix core is busy (on gfx950 a wave's VALU, LDS and buffer instructions
// co-issue with its own MFMAs): the next step's fragment reads after the
// first eight MFMAs, three VALU (the weight dequantization) after every one,
// the two LDS writes of the dequantized weight chunks and the step's share
// of the buffer loads spread in between.
#define LLMR_SGB(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
#define LLMR_SLOT_R LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x002, 3)
#define LLMR_SLOT_V LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 3)
#define LLMR_SLOT_L LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 3); LLMR_SGB(0x020, 1)
#define LLMR_SLOT_W LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 3); LLMR_SGB(0x200, 1)
#define LLMR_SLOT_RA LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x002, 5)
#define LLMR_SLOT_VA LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 5)
#define LLMR_SLOT_LA LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 5); LLMR_SGB(0x020, 1)
#define LLMR_SLOT_WA LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 5); LLMR_SGB(0x200, 1)
// the first step of a stage also computes the dequantization scales
#define LLMR_STEP_SCHEDULE_A                                                                \
    LLMR_SLOT_RA; LLMR_SLOT_RA; LLMR_SLOT_RA; LLMR_SLOT_RA; LLMR_SLOT_RA; LLMR_SLOT_RA;       \
    LLMR_SLOT_RA; LLMR_SLOT_RA; LLMR_SLOT_LA; LLMR_SLOT_VA; LLMR_SLOT_WA; LLMR_SLOT_LA;       \
    LLMR_SLOT_VA; LLMR_SLOT_WA; LLMR_SLOT_LA; LLMR_SLOT_LA
#define LLMR_STEP_SCHEDULE                                                                  \
    LLMR_SLOT_R; LLMR_SLOT_R; LLMR_SLOT_R; LLMR_SLOT_R; LLMR_SLOT_R; LLMR_SLOT_R;             \
    LLMR_SLOT_R; LLMR_SLOT_R; LLMR_SLOT_L; LLMR_SLOT_V; LLMR_SLOT_W; LLMR_SLOT_L;             \
    LLMR_SLOT_V; LLMR_SLOT_W; LLMR_SLOT_L; LLMR_SLOT_L

struct Frags {
    f16x8 x[4], w[4];
};

// silu(g) = g / (1 + e^-g) (llm.slang:1903), e^-g as 2^(-g log2 e)
__device__ __forceinline__ float silu(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// gelu (tanh form, lib/shaders/diffusion.slang:1103-1107) as
// 0.5 x (1 + tanh(u)) = x / (1 + e^(-2u)), u = 0.7978845608 (x + 0.044715 x^3)
__device__ __forceinline__ float gelu_tanh(float x) {
    const float u = 0.7978845608f * (x + 0.044715f * x * x * x);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * u));
}

// Output of the persistent kernel's tile accumulators (host-selected):
//   kEpiStore      Y[m, n] = acc
//   kEpiResidual   Y[m, n] += gate[n] * acc  (gate 1 when null)
//   kEpiSplitGelu  n < split: Y[m, n] = acc; n >= split: Y2[m, n - split] =
//                  16-bit gelu(acc)   (split % 8 == 0)
//   kEpiSplitSwiglu  tiles below split (split % 256 == 0): Y[m, n] = acc;
//                  the tiles past it are SwiGLU tiles of the weight image
//                  (256 rows: gate and up rows of 128 outputs, the
//                  arrangement of the SwiGLU kernel): Y2[m, o] = 16-bit
//                  silu(gate) * up, o < (N - split) / 2 (two-pass kernel)
// with row strides ldy (Y) and ldy2 (Y2).
constexpr uint32_t kEpiStore = 0, kEpiResidual = 1, kEpiSplitGelu = 2, kEpiSplitSwiglu = 3;

template <typename T>
__device__ __forceinline__ T pick(uint32_t p, T a, T b) {
    return p ? b : a;
}


// Head routing of one wave's 128 features n0w .. n0w + 127, one head of one
// Q/K/V slot (split % 128 == 0), for its 128 tokens, as qkv_heads_kernel
// computes it from the f32 GEMM output, bit for bit: per token the sum of
// the squares of its 64 pairs (2j, 2j + 1) in the same tree as that
// kernel's butterfly over pairs (a lane holds pairs j = 16 a + 4 g + 2 kh +
// e, so the levels across a, g are in the lane, the level across kh is the
// partner lane's, and the level across e comes last), x * rms * norm[f],
// pairs rotated by cos/sin[t, j], rounded to 16 bits into dst[head, t, f].
// A block's 32 tokens are consecutive rows of the RoPE tables, 8 KiB of
// each: they are DMA'd whole into lc / ls (the wave's own 8 KiB of LDS
// each), row r's logical 16-byte chunk c at physical chunk c ^ (r % 16), and
// each lane reads its pairs from there (read from memory per lane, a row per
// lane per load, the tables cost ~20 us per tile); a block's DMAs are issued
// before its sums of squares. The norm weights are read as scalar loads
// (both lanes' halves, selected by kh): as vector loads per block, their
// latency cost ~9 us per tile.
__device__ __forceinline__ void store_heads(f32x16 (&acc)[4][4], const HeadsEpi& h, uint32_t p, uint32_t M,
                                            uint32_t m0, uint32_t n0w, uint32_t wm, uint32_t l32, uint32_t kh,
                                            uint8_t* lc, uint8_t* ls) {
#pragma clang fp contract(off)
    typedef __attribute__((address_space(4))) const float cfloat;
    const uint32_t hs = n0w / 128u, slot = hs / h.n_heads, head = hs - slot * h.n_heads;
    uint16_t* const dst = (uint16_t*)(slot == 0 ? h.q : slot == 1 ? h.k : h.v) + (uint64_t)head * h.seq * 128u;
    const float* const nwp = slot == 0 ? pick(p, h.qn[0], h.qn[1]) : slot == 1 ? pick(p, h.kn[0], h.kn[1]) : nullptr;
    cfloat* const nw0 = (cfloat*)nwp;
    const bool rope = slot < 2 && h.cos != nullptr;
    const uint32_t row0 = __builtin_amdgcn_readfirstlane(pick(p, h.row0[0], h.row0[1]));
    const rsrc_t cr = make_rsrc(h.cos, rope ? (uint64_t)h.seq * 256u : 0u);
    const rsrc_t sr = make_rsrc(h.sin, rope ? (uint64_t)h.seq * 256u : 0u);
#pragma unroll
    for (int b = 0; b < 4; b++) {
        asm volatile("" : "+a"(acc[0][b]), "+a"(acc[1][b]), "+a"(acc[2][b]), "+a"(acc[3][b]));
        // the lane index opaque per block, so the 8 DMA and 16 LDS offsets
        // derived from it are computed here, not kept live across the tile
        // loop (which spilled the SwiGLU variants)
        uint32_t lane = l32 + 32u * kh;
        asm volatile("" : "+v"(lane));
        const uint32_t r32 = lane & 31u, sw = lane & 15u;
        // the norm pointer opaque per block too: its scalar loads stay here
        // (hoisted out of the tile loop, they took SGPRs the loop needs)
        cfloat* nw = nw0;
        asm volatile("" : "+s"(nw));
        const uint32_t m = m0 + wm * 128u + b * 32u + l32;
        const uint32_t t = row0 + m;  // < seq for m < M (host-checked)
        if (rope) {
            // DMA i: LDS rows 4 i .. 4 i + 3 (lane: row 4 i + lane / 16,
            // physical chunk lane % 16); rows past the tables read zero
            const uint32_t t0 = row0 + m0 + wm * 128u + b * 32u;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t r = 4u * i + (lane >> 4);
                const uint32_t vo = r * 256u + (((lane & 15u) ^ (r & 15u)) << 4);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(cr, (lds_void*)(lc + 1024u * i), 16, vo, t0 * 256u, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(ls + 1024u * i), 16, vo, t0 * 256u, 0, 0);
            }
        }
        float rms = 1.0f;
        if (nw) {
            float t4[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                float t3[2];
#pragma unroll
                for (int gl = 0; gl < 2; gl++) {
                    float t2[2];
#pragma unroll
                    for (int gh = 0; gh < 2; gh++) {
                        const int g = 2 * gh + gl;
                        float t1[2];
#pragma unroll
                        for (int al = 0; al < 2; al++) {
                            float sq[2];
#pragma unroll
                            for (int ah = 0; ah < 2; ah++) {
                                const float x0 = acc[2 * ah + al][b][4 * g + 2 * e];
                                const float x1 = acc[2 * ah + al][b][4 * g + 2 * e + 1];
                                sq[ah] = x0 * x0 + x1 * x1;
                            }
                            t1[al] = sq[0] + sq[1];
                        }
                        t2[gh] = t1[0] + t1[1];
                    }
                    t3[gl] = t2[0] + t2[1];
                }
                t4[e] = t3[0] + t3[1];
            }
            float t5[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(t4[e]), __float_as_uint(t4[e]),
                                                                false, false);
                t5[e] = t4[e] + __uint_as_float(kh ? r[0] : r[1]);  // plus the partner lane's
            }
            rms = 1.0f / __builtin_sqrtf((t5[0] + t5[1]) / 128.0f + h.eps);
        }
        if (rope) {  // this block's table rows have landed (its DMAs are the wave's only loads in flight)
            asm volatile("" ::: "memory");
            LLMR_WAIT_VMCNT(0);
            asm volatile("" ::: "memory");
        }
#pragma unroll
        for (int a = 0; a < 4; a++) {
            u32x2 pc[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                f32x4 x{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
                if (nw) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float wl = nw[32 * a + 8 * g + e], wh = nw[32 * a + 8 * g + 4 + e];
                        x[e] = (x[e] * rms) * (kh ? wh : wl);
                    }
                }
                if (rope) {  // pairs 16 a + 4 g + 2 kh + 0, 1: logical chunk 4 a + g of row l32, half kh
                    const uint32_t lo = r32 * 256u + (((4u * a + g) ^ sw) << 4) + 8u * kh;
                    const f32x2 c = *(const f32x2*)(lc + lo);
                    const f32x2 sn = *(const f32x2*)(ls + lo);
                    x = f32x4{x.x * c.x - x.y * sn.x, x.x * sn.x + x.y * c.x, x.z * c.y - x.w * sn.y,
                              x.z * sn.y + x.w * c.y};
                }
                pc[g] = h.out_bf16 ? u32x2{pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w)}
                                   : u32x2{pack_f16x2(x.x, x.y), pack_f16x2(x.z, x.w)};
            }
            // lane kh holds features 32 a + 8 g + 4 kh .. + 3; the two lanes
            // of a token trade pieces (kh = 0 gives its g = 1, 3 ones) so that
            // each stores 8 consecutive features, 16 bytes, per instruction
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const u32x2 give = kh ? pc[2 * q] : pc[2 * q + 1];
                u32x2 recv;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const auto r = __builtin_amdgcn_permlane32_swap(give[e], give[e], false, false);
                    recv[e] = kh ? r[0] : r[1];  // the partner lane's value
                }
                // kh = 0: features 32 a + 16 q + 0..7; kh = 1: + 8..15
                const u32x4 o = kh ? u32x4{recv.x, recv.y, pc[2 * q + 1].x, pc[2 * q + 1].y}
                                   : u32x4{pc[2 * q].x, pc[2 * q].y, recv.x, recv.y};
                if (m < M) *(u32x4*)(dst + (uint64_t)t * 128u + 32u * a + 16u * q + 8u * kh) = o;
            }
        }
#pragma unroll
        for (int a = 0; a < 4; a++) acc[a][b] = f32x16{};
        if (rope) {  // the reads of this block's rows are done before the next block's DMAs
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            asm volatile("" ::: "memory");
        }
    }
}

// HEADS (the two-pass kernel): head routing of the split epilogues, the
// wave's 8 KiB LDS regions lc, ls free for it (no DMA in flight into them).
template <bool SW, uint32_t EPI, bool HEADS = false>
__device__ __forceinline__ void store_tile_256(f32x16 (&acc)[4][4], float* Y, const float* gate, void* Y2v,
                                               uint32_t M, uint32_t N, uint32_t m0, uint32_t n0, uint32_t wm,
                                               uint32_t wn, uint32_t l32, uint32_t kh, uint32_t ldy, uint32_t ldy2,
                                               uint32_t split, uint32_t y2_bf16, const HeadsEpi* hd = nullptr,
                                               uint32_t p = 0, uint8_t* lc = nullptr, uint8_t* ls = nullptr) {
    if constexpr (HEADS && (EPI == kEpiSplitGelu || EPI == kEpiSplitSwiglu)) {
        // a wave's 128 features lie wholly below or above split (split % 128
        // == 0 with head routing; split % 256 == 0 for SwiGLU, where the
        // tiles past split hold other rows)
        if (hd->q != nullptr && n0 + wn * 128u < split) {
            store_heads(acc, *hd, p, M, m0, n0 + wn * 128u, wm, l32, kh, lc, ls);
            return;
        }
    }
    if constexpr (SW) {
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t m = m0 + wm * 128u + b * 32u + l32;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const uint32_t n = n0 + wn * 64u + a * 32u + 8u * g + 4u * kh;
                    f32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = silu(acc[a][b][4 * g + e]) * acc[a + 2][b][4 * g + e];
                    if (m < M && n < N) *(f32x4*)(Y + (uint64_t)m * ldy + n) = v;
                }
                acc[a][b] = f32x16{};
                acc[a + 2][b] = f32x16{};
            }
        return;
    }
    // The empty asm statement before each 32 x 32 block ("+a": the block's
    // accumulators are in AGPRs there and may change) keeps the compiler from
    // copying every accumulator into VGPRs at the top of the epilogue, which
    // spilled the gated-residual and split-SwiGLU variants to scratch; each
    // block is now copied out when it is stored.
    auto each = [&](auto&& f) __attribute__((always_inline)) {
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                asm volatile("" : "+a"(acc[a][b]));
                const uint32_t m = m0 + wm * 128u + b * 32u + l32;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const uint32_t nw = n0 + wn * 128u + a * 32u + 8u * g;
                    const uint32_t n = nw + 4u * kh;
                    if (m < M && n < N)
                        f(m, n, nw, f32x4{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                                          acc[a][b][4 * g + 3]});
                }
                acc[a][b] = f32x16{};
            }
    };
    if constexpr (EPI == kEpiSplitSwiglu) {
        if (n0 < split) {  // a plain tile (a uniform test: split % 256 == 0)
            each([&](uint32_t m, uint32_t n, uint32_t, f32x4 v) __attribute__((always_inline)) {
                *(f32x4*)(Y + (uint64_t)m * ldy + n) = v;
            });
            return;
        }
        // a SwiGLU tile: wave wn's 128 weight rows are gate rows 64 wn .. + 63
        // of the tile's 128 outputs (acc[0..1]) and the same outputs' up rows
        // (acc[2..3])
        uint16_t* const Y2 = (uint16_t*)Y2v;
        const uint32_t n_sw = (N - split) / 2u, o0 = (n0 - split) / 2u;
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                asm volatile("" : "+a"(acc[a][b]), "+a"(acc[a + 2][b]));
                const uint32_t m = m0 + wm * 128u + b * 32u + l32;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const uint32_t o = o0 + wn * 64u + a * 32u + 8u * g + 4u * kh;
                    f32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = silu(acc[a][b][4 * g + e]) * acc[a + 2][b][4 * g + e];
                    const u32x2 pk = y2_bf16 ? u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)}
                                             : u32x2{pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w)};
                    if (m < M && o < n_sw) *(u32x2*)(Y2 + (uint64_t)m * ldy2 + o) = pk;
                }
                acc[a][b] = f32x16{};
                acc[a + 2][b] = f32x16{};
            }
        return;
    }
    if constexpr (EPI == kEpiResidual) {
        each([&](uint32_t m, uint32_t n, uint32_t, f32x4 v) __attribute__((always_inline)) {
            f32x4* const h = (f32x4*)(Y + (uint64_t)m * ldy + n);
            const f32x4 gv = gate ? *(const f32x4*)(gate + n) : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
            *h = *h + gv * v;
        });
    } else if constexpr (EPI == kEpiSplitGelu) {
        uint16_t* const Y2 = (uint16_t*)Y2v;
        // A 32-feature block wholly past the split (a uniform test: split %
        // 8 == 0, nb uniform) with 16-byte aligned 16-bit rows: the two lanes
        // of a token (kh = 0, 1) trade 8-byte pieces so that each holds 8
        // consecutive features (16 bytes) twice, and a store instruction
        // writes 32-byte pieces of 32 rows instead of 16-byte ones (Flux
        // step 75.34 -> 75.13 ms, two runs each).
        const bool pair_ok = (ldy2 & 7u) == 0 && ((uintptr_t)Y2 & 15u) == 0;
        auto pack16 = [&](f32x4 v) __attribute__((always_inline)) {
            const f32x4 gl{gelu_tanh(v.x), gelu_tanh(v.y), gelu_tanh(v.z), gelu_tanh(v.w)};
            if (y2_bf16) {
                typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
                return u32x2{__builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)gl.x, (__bf16)gl.y}),
                             __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)gl.z, (__bf16)gl.w})};
            }
            return u32x2{pack_f16x2(gl.x, gl.y), pack_f16x2(gl.z, gl.w)};
        };
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint32_t nb = n0 + wn * 128u + a * 32u;  // the block's first feature (uniform)
            const bool paired = pair_ok && nb >= split && nb + 32u <= N;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                asm volatile("" : "+a"(acc[a][b]));
                const uint32_t m = m0 + wm * 128u + b * 32u + l32;
                if (paired) {
                    u32x2 pc[4];
#pragma unroll
                    for (int g = 0; g < 4; g++)
                        pc[g] = pack16(f32x4{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                                             acc[a][b][4 * g + 3]});
                    // lane kh holds features 8 g + 4 kh .. +3; kh = 0 gives its
                    // g = 1, 3 pieces for the partner's g = 0, 2 pieces
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const u32x2 give = kh ? pc[2 * t] : pc[2 * t + 1];
                        u32x2 recv;
#pragma unroll
                        for (int e = 0; e < 2; e++) {
                            const auto r = __builtin_amdgcn_permlane32_swap(give[e], give[e], false, false);
                            recv[e] = kh ? r[0] : r[1];  // the partner lane's value
                        }
                        // kh = 0: features 16 t + 0..7; kh = 1: 16 t + 8..15
                        const u32x4 o = kh ? u32x4{recv.x, recv.y, pc[2 * t + 1].x, pc[2 * t + 1].y}
                                           : u32x4{pc[2 * t].x, pc[2 * t].y, recv.x, recv.y};
                        if (m < M) *(u32x4*)(Y2 + (uint64_t)m * ldy2 + (nb + 16u * t + 8u * kh - split)) = o;
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const uint32_t nw = nb + 8u * g;
                        const uint32_t n = nw + 4u * kh;
                        if (m >= M || n >= N) continue;
                        const f32x4 v{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                                      acc[a][b][4 * g + 3]};
                        if (nw < split)
                            *(f32x4*)(Y + (uint64_t)m * ldy + n) = v;
                        else
                            *(u32x2*)(Y2 + (uint64_t)m * ldy2 + (n - split)) = pack16(v);
                    }
                }
                acc[a][b] = f32x16{};
            }
        }
    } else {
        each([&](uint32_t m, uint32_t n, uint32_t, f32x4 v) __attribute__((always_inline)) {
            *(f32x4*)(Y + (uint64_t)m * ldy + n) = v;
        });
    }
}

}  // namespace
}  // namespace llmr
