// gemm_q.hip - GGUF Q8_0 / Q4_K dequant-GEMM on gfx950 matrix cores.
//
//   Y[m, n] = sum_k X[m, k] * W[row_offset + n, k]     (f32 out, row stride N)
//
// Semantics of batch_matmul_q8 (llm.slang:1613-1767) and batch_matmul_q4k
// (llm.slang:2264-2365), selected as in dispatch_batch_matmul
// (dependencies/zimage.c3l/dit.c3:1198-1301).
//
// Design (one 256-thread workgroup = 4 wave64s per BM x BN output tile):
//  * K is walked in stages of 64 (two Q8_0 blocks, or one quarter of a Q4_K
//    superblock: qs bytes [32j, 32j+32) = sub-blocks 2j and 2j+1).
//  * Each stage, every thread loads its share of the activation tile (f32,
//    f16 or bf16 -> fp16) and of the raw packed weight tile from HBM with
//    16-byte loads, dequantizes the weights in registers (Q8_0: RN16(d*q),
//    the reference's operand; Q4_K: RN16(d*sc*q - dmin*mn)) and writes both
//    tiles to LDS as fp16 [rows][64] with a XOR swizzle of the 16-byte
//    chunks so the fragment reads are bank-conflict free.
//  * Loads for stage s+1 are issued before the matrix work of stage s and the
//    LDS tiles are double buffered: one barrier per stage.
//  * Each wave owns a (BN/2) x (BM/2) sub-tile and accumulates it in f32 with
//    v_mfma_f32_32x32x16_f16 (W rows as the A operand, X rows as B), so each
//    lane holds 4 consecutive output features of one token per group and
//    the epilogue writes 16-byte stores.
//  * Within a 32-wide K chunk the MFMA's logical k index is permuted (lane
//    half kh, step s, element i -> k = 16kh + 8s + i) identically for both
//    operands, so every fragment is one 16-byte LDS read.
//  * Workgroups are remapped so the tiles one XCD runs concurrently share
//    weight and activation rows in that XCD's L2.
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

constexpr int kBK = 64;  // K per stage

// 16-byte chunk c (0..7) of LDS row r (128-byte rows). gfx950's LDS has 64
// four-byte banks, so two rows share a 256-byte bank line; XOR-ing the chunk
// with (r >> 1) & 7 makes the 16 rows of a 16-lane fragment read land on 16
// distinct bank quads.
__device__ __forceinline__ uint32_t lds_off(uint32_t r, uint32_t c) {
    return r * 128u + ((c ^ ((r >> 1) & 7u)) << 4);
}

template <uint32_t XT>
struct XLoad;

// bf16 / f16 activations: one 16-byte load per LDS chunk.
template <>
struct XLoad<kGgmlBF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const void* x, uint64_t elem, bool ok) {
        v = ok ? *(const u32x4*)((const uint16_t*)x + elem) : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ u32x4 to_f16() const {
        return u32x4{bf16x2_to_f16x2(v.x), bf16x2_to_f16x2(v.y), bf16x2_to_f16x2(v.z),
                     bf16x2_to_f16x2(v.w)};
    }
};
template <>
struct XLoad<kGgmlF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const void* x, uint64_t elem, bool ok) {
        v = ok ? *(const u32x4*)((const uint16_t*)x + elem) : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ u32x4 to_f16() const { return v; }
};
// f32 activations: two 16-byte loads per LDS chunk, rounded to fp16 as the
// reference's float16_t(v) (llm.slang:1673).
template <>
struct XLoad<kGgmlF32> {
    f32x4 a, b;
    __device__ __forceinline__ void load(const void* x, uint64_t elem, bool ok) {
        const float* p = (const float*)x + elem;
        a = ok ? *(const f32x4*)p : f32x4{0, 0, 0, 0};
        b = ok ? *(const f32x4*)(p + 4) : f32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ u32x4 to_f16() const {
        return u32x4{pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y),
                     pack_f16x2(b.z, b.w)};
    }
};

// Weight stage loaders. A "unit" is the part of one weight row's stage that
// one thread loads and dequantizes.
template <uint32_t WT>
struct WLoad;

// Q8_0: unit = one row's two blocks of the stage, 68 bytes = 17 dwords
// (dword aligned because K % 64 == 0 makes the row length a multiple of 68).
template <>
struct WLoad<kGgmlQ8_0> {
    static constexpr int kUnitsPerRow = 1;
    u32x4 a, b, c, d;
    uint32_t e;
    __device__ __forceinline__ void load(const uint8_t* w, uint64_t row_bytes, uint32_t row,
                                         uint32_t unit, uint32_t k0, bool ok) {
        (void)unit;
        if (!ok) {
            a = b = c = d = u32x4{0, 0, 0, 0};
            e = 0;
            return;
        }
        const uint8_t* p = w + (uint64_t)row * row_bytes + (uint64_t)(k0 / 32) * 34;
        a = *(const u32x4_a4*)(p + 0);
        b = *(const u32x4_a4*)(p + 16);
        c = *(const u32x4_a4*)(p + 32);
        d = *(const u32x4_a4*)(p + 48);
        e = *(const uint32_t*)(p + 64);
    }
    // Writes chunks 0..7 of LDS row r (k 0..31 from block 0, 32..63 from block 1).
    __device__ __forceinline__ void store(uint8_t* lds, uint32_t r, uint32_t unit) const {
        (void)unit;
        const uint32_t wd[17] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x,
                                 c.y, c.z, c.w, d.x, d.y, d.z, d.w, e};
        // block 0: scale = bytes 0-1, quants = bytes 2..33 (re-aligned by 2 bytes)
        const _Float16 d0 = (_Float16)f16_bits_to_f32(wd[0] & 0xffffu);
        const f16x2 d02 = {d0, d0};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            const uint32_t q0 = __builtin_amdgcn_alignbyte(wd[2 * ch + 1], wd[2 * ch], 2);
            const uint32_t q1 = __builtin_amdgcn_alignbyte(wd[2 * ch + 2], wd[2 * ch + 1], 2);
            const f16x4 lo = q8x4_to_f16(q0, d02);
            const f16x4 hi = q8x4_to_f16(q1, d02);
            f16x8 v;
            v.s0 = lo.x; v.s1 = lo.y; v.s2 = lo.z; v.s3 = lo.w;
            v.s4 = hi.x; v.s5 = hi.y; v.s6 = hi.z; v.s7 = hi.w;
            *(f16x8*)(lds + lds_off(r, ch)) = v;
        }
        // block 1: scale = bytes 34-35 (high half of dword 8), quants = dwords 9..16
        const _Float16 d1 = (_Float16)f16_bits_to_f32(wd[8] >> 16);
        const f16x2 d12 = {d1, d1};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            const f16x4 lo = q8x4_to_f16(wd[9 + 2 * ch], d12);
            const f16x4 hi = q8x4_to_f16(wd[10 + 2 * ch], d12);
            f16x8 v;
            v.s0 = lo.x; v.s1 = lo.y; v.s2 = lo.z; v.s3 = lo.w;
            v.s4 = hi.x; v.s5 = hi.y; v.s6 = hi.z; v.s7 = hi.w;
            *(f16x8*)(lds + lds_off(r, 4 + ch)) = v;
        }
    }
};

// Q4_K: unit = (row, half c2 of the stage's 32 qs bytes): 16 qs bytes give
// 16 low nibbles (k = 16*c2 + 0..15, sub-block 2j) and 16 high nibbles
// (k = 32 + 16*c2 + 0..15, sub-block 2j+1); plus the 16-byte block header.
template <>
struct WLoad<kGgmlQ4K> {
    static constexpr int kUnitsPerRow = 2;
    u32x4 hdr, qs;
    __device__ __forceinline__ void load(const uint8_t* w, uint64_t row_bytes, uint32_t row,
                                         uint32_t unit, uint32_t k0, bool ok) {
        if (!ok) {
            hdr = qs = u32x4{0, 0, 0, 0};
            return;
        }
        const uint8_t* p = w + (uint64_t)row * row_bytes + (uint64_t)(k0 / 256) * 144;
        const uint32_t j = (k0 % 256) / 64;
        hdr = *(const u32x4*)p;
        qs = *(const u32x4*)(p + 16 + 32 * j + 16 * unit);
    }
    __device__ __forceinline__ void store(uint8_t* lds, uint32_t r, uint32_t unit, uint32_t k0) const {
        const uint32_t j = (k0 % 256) / 64;
        const float d = f16_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(hdr.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(2 * j, hdr.y, hdr.z, hdr.w, sc0, mn0);
        q4k_scale_min(2 * j + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
        const float dsc0 = d * (float)sc0, dmn0 = dmin * (float)mn0;
        const float dsc1 = d * (float)sc1, dmn1 = dmin * (float)mn1;
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l4 = q[i] & 0x0f0f0f0fu;
            const uint32_t h4 = (q[i] >> 4) & 0x0f0f0f0fu;
            lo[2 * i] = q4_pair(l4, 0x04010400u, dsc0, dmn0);
            lo[2 * i + 1] = q4_pair(l4, 0x04030402u, dsc0, dmn0);
            hi[2 * i] = q4_pair(h4, 0x04010400u, dsc1, dmn1);
            hi[2 * i + 1] = q4_pair(h4, 0x04030402u, dsc1, dmn1);
        }
        *(u32x4*)(lds + lds_off(r, 2 * unit)) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        *(u32x4*)(lds + lds_off(r, 2 * unit + 1)) = u32x4{lo[4], lo[5], lo[6], lo[7]};
        *(u32x4*)(lds + lds_off(r, 4 + 2 * unit)) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        *(u32x4*)(lds + lds_off(r, 5 + 2 * unit)) = u32x4{hi[4], hi[5], hi[6], hi[7]};
    }
};

// Tile id -> (tile_m, tile_n): consecutive ids on one XCD (hardware deals
// workgroups round-robin to the 8 XCDs) get a contiguous range of tiles,
// walked in groups of kGroupM m-tiles so concurrent tiles share W rows.
__device__ __forceinline__ void map_tile(uint32_t bid, uint32_t tiles_m, uint32_t tiles_n,
                                         uint32_t& tm, uint32_t& tn) {
    constexpr uint32_t kXcd = 8, kGroupM = 8;
    const uint32_t total = tiles_m * tiles_n;
    uint32_t L = bid;
    if (total % kXcd == 0) L = (bid % kXcd) * (total / kXcd) + bid / kXcd;
    const uint32_t per_group = kGroupM * tiles_n;
    const uint32_t g = L / per_group;
    const uint32_t first_m = g * kGroupM;
    const uint32_t gsize = min(tiles_m - first_m, kGroupM);
    const uint32_t in = L % per_group;
    tm = first_m + in % gsize;
    tn = in / gsize;
}

template <uint32_t WT, uint32_t XT, int BM, int BN>
__global__ void __launch_bounds__(256, (BM * BN >= 256 * 256) ? 1 : 2)
gemm_q_mfma(const uint8_t* __restrict__ W, const void* __restrict__ X, float* __restrict__ Y,
            uint32_t N, uint32_t K, uint32_t M, uint32_t row_offset, uint32_t tiles_m,
            uint32_t tiles_n) {
    constexpr int WM = BM / 2, WN = BN / 2;  // per-wave tile (tokens x features)
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr uint32_t A_BYTES = BM * kBK * 2, B_BYTES = BN * kBK * 2;
    constexpr uint32_t STAGE = A_BYTES + B_BYTES;
    constexpr int X_PER_T = BM * 8 / 256;                        // activation chunks per thread
    constexpr int W_UNITS = BN * WLoad<WT>::kUnitsPerRow;        // weight units per stage
    constexpr int W_PER_T = (W_UNITS + 255) / 256;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const uint32_t wm = wave & 1u, wn = wave >> 1;

    uint32_t tile_m, tile_n;
    map_tile(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
    const uint32_t m0 = tile_m * BM, n0 = tile_n * BN;
    const uint64_t row_bytes = (WT == kGgmlQ8_0) ? (uint64_t)(K / 32) * 34 : (uint64_t)(K / 256) * 144;
    const uint8_t* Wt = W + (uint64_t)row_offset * row_bytes;
    const uint32_t n_stages = K / kBK;

    XLoad<XT> xl[X_PER_T];
    WLoad<WT> wl[W_PER_T];

    auto load_stage = [&](uint32_t s) {
        const uint32_t k0 = s * kBK;
#pragma unroll
        for (int i = 0; i < X_PER_T; i++) {
            const uint32_t r = (tid >> 3) + 32u * i, c = tid & 7u;
            const uint32_t m = m0 + r;
            xl[i].load(X, (uint64_t)m * K + k0 + 8u * c, m < M);
        }
#pragma unroll
        for (int i = 0; i < W_PER_T; i++) {
            const uint32_t u = tid + 256u * i;
            const uint32_t r = u / WLoad<WT>::kUnitsPerRow, unit = u % WLoad<WT>::kUnitsPerRow;
            const bool ok = (u < (uint32_t)W_UNITS) && (n0 + r < N);
            wl[i].load(Wt, row_bytes, n0 + r, unit, k0, ok);
        }
    };
    auto store_stage = [&](uint32_t s, uint32_t buf) {
        uint8_t* As = smem + buf * STAGE;
        uint8_t* Bs = As + A_BYTES;
#pragma unroll
        for (int i = 0; i < X_PER_T; i++) {
            const uint32_t r = (tid >> 3) + 32u * i, c = tid & 7u;
            *(u32x4*)(As + lds_off(r, c)) = xl[i].to_f16();
        }
#pragma unroll
        for (int i = 0; i < W_PER_T; i++) {
            const uint32_t u = tid + 256u * i;
            if (u < (uint32_t)W_UNITS) {
                const uint32_t r = u / WLoad<WT>::kUnitsPerRow, unit = u % WLoad<WT>::kUnitsPerRow;
                if constexpr (WT == kGgmlQ4K)
                    wl[i].store(Bs, r, unit, s * kBK);
                else
                    wl[i].store(Bs, r, unit);
            }
        }
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; a++)
#pragma unroll
        for (int b = 0; b < TM; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.0f;

    load_stage(0);
    store_stage(0, 0);
    __syncthreads();

    for (uint32_t s = 0; s < n_stages; s++) {
        const uint32_t buf = s & 1u;
        if (s + 1 < n_stages) load_stage(s + 1);
        const uint8_t* As = smem + buf * STAGE;
        const uint8_t* Bs = As + A_BYTES;
#pragma unroll
        for (int c = 0; c < 2; c++) {
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const uint32_t ch = 4u * c + 2u * kh + st;
                f16x8 xf[TM], wf[TN];
#pragma unroll
                for (int b = 0; b < TM; b++) {
                    const uint32_t r = wm * WM + b * 32 + l32;
                    xf[b] = *(const f16x8*)(As + lds_off(r, ch));
                }
#pragma unroll
                for (int a = 0; a < TN; a++) {
                    const uint32_t r = wn * WN + a * 32 + l32;
                    wf[a] = *(const f16x8*)(Bs + lds_off(r, ch));
                }
#pragma unroll
                for (int a = 0; a < TN; a++)
#pragma unroll
                    for (int b = 0; b < TM; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[a], xf[b], acc[a][b], 0, 0, 0);
            }
        }
        if (s + 1 < n_stages) store_stage(s + 1, buf ^ 1u);
        __syncthreads();
    }

    // Epilogue: lane holds token m = .. + l32 and features n = 8g + 4kh + 0..3.
    const bool vec_ok = (N % 4u) == 0u;
#pragma unroll
    for (int a = 0; a < TN; a++)
#pragma unroll
        for (int b = 0; b < TM; b++) {
            const uint32_t m = m0 + wm * WM + b * 32 + l32;
            if (m >= M) continue;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t n = n0 + wn * WN + a * 32 + 8 * g + 4 * kh;
                float* yp = Y + (uint64_t)m * N + n;
                const f32x4 v = {acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                                 acc[a][b][4 * g + 3]};
                if (vec_ok && n + 3 < N) {
                    *(f32x4*)yp = v;
                } else {
                    if (n < N) yp[0] = v.x;
                    if (n + 1 < N) yp[1] = v.y;
                    if (n + 2 < N) yp[2] = v.z;
                    if (n + 3 < N) yp[3] = v.w;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// 256 x 256 tile kernel for 16-bit activations, software pipelined.
//
// Same tile mapping, LDS row layout and MFMA k-permutation as gemm_q_mfma.
// The activations are multiplied in their own type: bf16 activations with
// v_mfma_f32_32x32x16_bf16 (converting them to fp16 would overflow above
// 65504), f16 activations with the f16 instruction; the weights are
// dequantized to that type (bf16: RN_bf16 of the reference's f32 dequant
// value; f16: the fp16 operand of gemm_q_mfma). Restructured so the matrix
// cores are not left waiting for the byte work:
//  * the activation tile goes from HBM straight into LDS (buffer_load ... lds,
//    16 bytes per lane; the per-lane source address is permuted so the fixed
//    lane*16 LDS placement realizes the bank swizzle), into a 3-slot ring
//    fetched two stages ahead - no registers, no VALU;
//  * the weight tile is fetched into two register sets (two stages ahead),
//    dequantized into a double-buffered LDS tile while the previous stage is
//    multiplied (the VALU work is interleaved with the MFMAs);
//  * all global reads use buffer descriptors whose size ends at the last
//    valid row of the tile: the hardware returns zeros past it, so the loop
//    has no bounds branches; reads past the last stage land in LDS that is
//    never multiplied;
//  * LDS is 3 x 32 KiB (activations) + 2 x 32 KiB (weights) = 160 KiB.
// ---------------------------------------------------------------------------

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint64_t bytes) {
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
// s_waitcnt vmcnt(n) leaving the LDS and export counters unconstrained
// (gfx9 encoding: vmcnt[3:0] | expcnt << 4 | lgkmcnt << 8 | vmcnt[5:4] << 14).
#define LLMR_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))

// Workgroup barrier for the pipelined loop: this wave's LDS writes are done
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

// Q4_K nibbles -> packed bf16 of the reference's f32 value d*sc*q - dmin*mn
// (q exact via the 1024+q half, f32 FMA, then RNE to bf16).
__device__ __forceinline__ uint32_t q4_pair_bf16(uint32_t nib, uint32_t sel, float dsc, float dmn) {
    const f16x2 bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    const f16x2 q = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, nib, sel)) - bias;
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t r;
    r.x = (__bf16)__builtin_fmaf((float)q.x, dsc, -dmn);
    r.y = (__bf16)__builtin_fmaf((float)q.y, dsc, -dmn);
    return __builtin_bit_cast(uint32_t, r);
}
// Four Q8_0 quants -> two dwords of packed bf16 RN_bf16(d*q) (d*q exact in f32).
__device__ __forceinline__ u32x2 q8x4_to_bf16(uint32_t w, float d) {
    const uint32_t x = w ^ 0x80808080u;
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2 a = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) - bias;
    const f16x2 b = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) - bias;
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t r0, r1;
    r0.x = (__bf16)((float)a.x * d);
    r0.y = (__bf16)((float)a.y * d);
    r1.x = (__bf16)((float)b.x * d);
    r1.y = (__bf16)((float)b.y * d);
    return u32x2{__builtin_bit_cast(uint32_t, r0), __builtin_bit_cast(uint32_t, r1)};
}

// Eight Q8_0 quants (two dwords) -> one 16-byte chunk of operand type OT.
template <uint32_t OT>
__device__ __forceinline__ u32x4 q8x8_operand(uint32_t q0, uint32_t q1, float d, f16x2 d2) {
    if constexpr (OT == kGgmlBF16) {
        const u32x2 lo = q8x4_to_bf16(q0, d), hi = q8x4_to_bf16(q1, d);
        return u32x4{lo.x, lo.y, hi.x, hi.y};
    } else {
        const f16x4 lo = q8x4_to_f16(q0, d2), hi = q8x4_to_f16(q1, d2);
        return __builtin_bit_cast(u32x4, f16x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
    }
}

// One thread's weight unit of one stage, dequantized to operand type OT
// (kGgmlF16 or kGgmlBF16). 512 threads cover the 256-row tile; 16
// consecutive lanes take 16 consecutive rows with the same chunk set, so
// their 16-byte LDS writes hit 16 distinct bank quads:
//   row = (tid & 15) + 16 * (tid >> 5), part = (tid >> 4) & 1.
__device__ __forceinline__ uint32_t wunit_row(uint32_t tid) { return (tid & 15u) + 16u * (tid >> 5); }
__device__ __forceinline__ uint32_t wunit_part(uint32_t tid) { return (tid >> 4) & 1u; }

template <uint32_t WT, uint32_t OT>
struct WUnit;

// Q4_K: part p = half of the stage's 32 qs bytes of the row: 16 low nibbles
// (k = 16p + 0..15, sub-block 2j) and 16 high nibbles (k = 32 + 16p + 0..15,
// sub-block 2j+1), plus the 16-byte block header.
template <uint32_t OT>
struct WUnit<kGgmlQ4K, OT> {
    static constexpr int kLoads = 2;
    u32x4 hdr, qs;
    // `end` (the descriptor size) replaces the stage offset of a padding stage
    // past the last one, so every load of it returns zeros.
    __device__ __forceinline__ void load(rsrc_t r, uint32_t voff, uint32_t k0, bool live, uint32_t end) {
        const uint32_t sh = live ? (k0 >> 8) * 144u : end;
        const uint32_t sq = live ? sh + 16u + 32u * ((k0 >> 6) & 3u) : end;
        hdr = bload16(r, voff, sh);
        qs = bload16(r, voff + 16u * wunit_part(threadIdx.x), sq);
    }
    // LDS offsets of the 4 destination chunks 2p, 2p+1, 4+2p, 5+2p of the row
    __device__ __forceinline__ static void offsets(uint32_t (&off)[4]) {
        const uint32_t r = wunit_row(threadIdx.x), p = wunit_part(threadIdx.x);
        off[0] = lds_off(r, 2u * p);
        off[1] = lds_off(r, 2u * p + 1u);
        off[2] = lds_off(r, 4u + 2u * p);
        off[3] = lds_off(r, 5u + 2u * p);
    }
    __device__ __forceinline__ void store(uint8_t* lds, uint32_t k0, const uint32_t (&off)[4]) const {
        const uint32_t j = (k0 >> 6) & 3u;
        const float d = f16_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(hdr.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(2 * j, hdr.y, hdr.z, hdr.w, sc0, mn0);
        q4k_scale_min(2 * j + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
        const float dsc0 = d * (float)sc0, dmn0 = dmin * (float)mn0;
        const float dsc1 = d * (float)sc1, dmn1 = dmin * (float)mn1;
        const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t l4 = q[e] & 0x0f0f0f0fu;
            const uint32_t h4 = (q[e] >> 4) & 0x0f0f0f0fu;
            if constexpr (OT == kGgmlBF16) {
                lo[2 * e] = q4_pair_bf16(l4, 0x04010400u, dsc0, dmn0);
                lo[2 * e + 1] = q4_pair_bf16(l4, 0x04030402u, dsc0, dmn0);
                hi[2 * e] = q4_pair_bf16(h4, 0x04010400u, dsc1, dmn1);
                hi[2 * e + 1] = q4_pair_bf16(h4, 0x04030402u, dsc1, dmn1);
            } else {
                lo[2 * e] = q4_pair(l4, 0x04010400u, dsc0, dmn0);
                lo[2 * e + 1] = q4_pair(l4, 0x04030402u, dsc0, dmn0);
                hi[2 * e] = q4_pair(h4, 0x04010400u, dsc1, dmn1);
                hi[2 * e + 1] = q4_pair(h4, 0x04030402u, dsc1, dmn1);
            }
        }
        *(u32x4*)(lds + off[0]) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        *(u32x4*)(lds + off[1]) = u32x4{lo[4], lo[5], lo[6], lo[7]};
        *(u32x4*)(lds + off[2]) = u32x4{hi[0], hi[1], hi[2], hi[3]};
        *(u32x4*)(lds + off[3]) = u32x4{hi[4], hi[5], hi[6], hi[7]};
    }
};

// Q8_0: part p = block p of the stage's two blocks (k = 32p + 0..31). The 9
// dwords loaded from the dword-aligned start hold the block: p = 0 starts at
// the stage's byte 0 (scale in the low half of dword 0, quants from byte 2),
// p = 1 at byte 34 (loaded from byte 32: scale in the high half of dword 0,
// quants in dwords 1..8).
template <uint32_t OT>
struct WUnit<kGgmlQ8_0, OT> {
    static constexpr int kLoads = 3;
    u32x4 a, b;
    uint32_t c;
    __device__ __forceinline__ void load(rsrc_t r, uint32_t voff, uint32_t k0, bool live, uint32_t end) {
        const uint32_t s = live ? (k0 >> 5) * 34u : end;
        const uint32_t v = voff + 32u * wunit_part(threadIdx.x);
        a = bload16(r, v, s);
        b = bload16(r, v + 16u, s);
        c = bload4(r, v + 32u, s);
    }
    __device__ __forceinline__ static void offsets(uint32_t (&off)[4]) {
        const uint32_t r = wunit_row(threadIdx.x), p = wunit_part(threadIdx.x);
#pragma unroll
        for (int k = 0; k < 4; k++) off[k] = lds_off(r, 4u * p + k);
    }
    __device__ __forceinline__ void store(uint8_t* lds, uint32_t k0, const uint32_t (&off)[4]) const {
        (void)k0;
        const bool p1 = wunit_part(threadIdx.x) != 0;
        const uint32_t wd[9] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c};
        const float d = f16_bits_to_f32(p1 ? (wd[0] >> 16) : (wd[0] & 0xffffu));
        const _Float16 h = (_Float16)d;
        const f16x2 d2 = {h, h};
        uint32_t qd[8];
#pragma unroll
        for (int i = 0; i < 8; i++) qd[i] = p1 ? wd[i + 1] : __builtin_amdgcn_alignbyte(wd[i + 1], wd[i], 2);
#pragma unroll
        for (int ch = 0; ch < 4; ch++) *(u32x4*)(lds + off[ch]) = q8x8_operand<OT>(qd[2 * ch], qd[2 * ch + 1], d, d2);
    }
};

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

// 512 threads = 8 waves = 2 per SIMD (one wave's LDS and barrier stalls are
// covered by the other's MFMAs; on gfx950 vector ALU work does not overlap
// matrix work on the same SIMD, so the dequant cost is kept to a minimum
// instead). Wave tile 128 tokens x 64 features (wave grid 2 x 4).
template <uint32_t WT, uint32_t XT>
__global__ void __launch_bounds__(512, 1)
gemm_q_pipe(const uint8_t* __restrict__ W, const void* __restrict__ X, float* __restrict__ Y, uint32_t N,
            uint32_t K, uint32_t M, uint32_t row_offset, uint32_t tiles_m, uint32_t tiles_n) {
    static_assert(XT == kGgmlF16 || XT == kGgmlBF16, "16-bit activations only");
    constexpr int BM = 256, BN = 256, WM = 128, WN = 64, TM = 4, TN = 2;
    constexpr uint32_t TILE = 256u * 128u;  // bytes of one 256-row x 64-wide 16-bit tile
    constexpr int W_LOADS = WUnit<WT, XT>::kLoads;
    constexpr int X_DMAS = 4;  // 1 KiB activation DMAs per wave per stage
    // three separate arrays (not one indexed ring) so the compiler can prove a
    // DMA into one slot does not alias reads of another and does not wait for it
    __shared__ __attribute__((aligned(16))) uint8_t X0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t X1[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t X2[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t W0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t W1[TILE];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const uint32_t wm = wave & 1u, wn = wave >> 1;

    uint32_t tile_m, tile_n;
    map_tile(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
    const uint32_t m0 = tile_m * BM, n0 = tile_n * BN;
    const uint32_t rb = (WT == kGgmlQ8_0) ? (K / 32u) * 34u : (K / 256u) * 144u;
    // descriptor sizes end at the last valid row; the host guarantees they and
    // every offset used below fit in 31 bits
    const uint32_t x_end = (M - m0) * K * 2u;
    const uint32_t w_end = (N - n0) * rb;
    const rsrc_t xr = make_rsrc((const uint8_t*)X + (uint64_t)m0 * K * 2u, x_end);
    const rsrc_t wr = make_rsrc(W + (uint64_t)(row_offset + n0) * rb, w_end);
    const uint32_t n_stages = K / kBK;

    // activation DMA: wave w fills rows 32w .. 32w+31 of a slot, 8 rows (1 KiB)
    // per instruction; lane l lands at byte 16l of the instruction's block,
    // i.e. row 32w + 8i + l/8, physical chunk l%8, so it fetches logical chunk
    // (l%8) ^ swizzle(row).
    uint32_t xvoff[X_DMAS];
#pragma unroll
    for (int i = 0; i < X_DMAS; i++) {
        const uint32_t row = 32u * wave + 8u * i + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ ((row >> 1) & 7u);
        xvoff[i] = row * K * 2u + c * 16u;
    }
    auto dma_x = [&](uint32_t stage, uint8_t* Xslot) {
        uint8_t* slot = Xslot + 32u * wave * 128u;
        const uint32_t soff = stage < n_stages ? stage * kBK * 2u : x_end;
#pragma unroll
        for (int i = 0; i < X_DMAS; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(slot + 1024u * i), 16, xvoff[i], soff, 0, 0);
    };

    const uint32_t wvoff = wunit_row(tid) * rb;
    WUnit<WT, XT> wu0, wu1;
    auto wload = [&](WUnit<WT, XT>& u, uint32_t stage) {
        u.load(wr, wvoff, stage * kBK, stage < n_stages, w_end);
    };
    uint32_t stoff[4];
    WUnit<WT, XT>::offsets(stoff);

    // Fragment addresses. Every row block starts at a multiple of 32 rows, so
    // the swizzle term (row >> 1) & 7 depends only on the lane: each operand
    // needs one lane offset per 16-wide k step t (chunk 4(t>>1) + 2kh + (t&1));
    // the buffer and the row block are compile-time displacements.
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t ch = 4u * (t >> 1) + 2u * kh + (t & 1);
        xoff[t] = lds_off(wm * WM + l32, ch);
        woff[t] = lds_off(wn * WN + l32, ch);
    }

    f32x16 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; a++)
#pragma unroll
        for (int b = 0; b < TM; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) acc[a][b][i] = 0.0f;

    // Multiply stage s (activations As, weights Bs) while dequantizing `u`
    // (the weights of stage s+1) into Bn.
    // The fragments of a k step are read right before its MFMAs: the other
    // wave on the SIMD covers the LDS latency.
    auto stage = [&](uint32_t s, const uint8_t* As, const uint8_t* Bs, const WUnit<WT, XT>& u, uint8_t* Bn) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            f16x8 xf[TM], wf[TN];
#pragma unroll
            for (int b = 0; b < TM; b++) xf[b] = *(const f16x8*)(As + b * 32 * 128 + xoff[t]);
#pragma unroll
            for (int a = 0; a < TN; a++) wf[a] = *(const f16x8*)(Bs + a * 32 * 128 + woff[t]);
            if (t == 1) u.store(Bn, (s + 1) * kBK, stoff);
#pragma unroll
            for (int a = 0; a < TN; a++)
#pragma unroll
                for (int b = 0; b < TM; b++) acc[a][b] = mfma16<XT>(wf[a], xf[b], acc[a][b]);
            // keep the next step's fragment reads below this step's MFMAs: at
            // most one step of fragments is live (no spills, whose reloads
            // would wait on every load in flight)
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // prologue: activations of stages 0 and 1 in flight to LDS, weights of
    // stage 0 dequantized into W0, weights of stages 1 and 2 in registers
    dma_x(0, X0);
    dma_x(1, X1);
    wload(wu0, 0);
    wload(wu1, 1);
    wu0.store(W0, 0, stoff);
    wload(wu0, 2);
    LLMR_STAGE_BARRIER(X_DMAS + 2 * W_LOADS);  // stage-0 activations have landed

    // Stage t = s + i: DMA the activations of stage t+2 into the free slot,
    // multiply stage t while storing the weights of stage t+1, fetch the
    // weights of stage t+3; then wait until stage t+1's activations have
    // landed (only the DMAs and weight fetches issued after them may stay in
    // flight) and barrier. Unrolled by 6 = lcm(3 activation slots, 2 weight
    // buffers) so every LDS buffer is a compile-time choice; the stage count
    // is padded to a multiple of 6 with all-zero stages (their loads start at
    // the descriptor end) instead of exiting mid-body.
#define LLMR_PIPE_ITER(i, XC, XD, WC, WN_, U)                 \
    dma_x(s + (i) + 2, XD);                                   \
    stage(s + (i), XC, WC, U, WN_);                           \
    wload(U, s + (i) + 3);                                    \
    LLMR_STAGE_BARRIER(X_DMAS + 2 * W_LOADS);
    for (uint32_t s = 0; s < n_stages; s += 6) {
        LLMR_PIPE_ITER(0, X0, X2, W0, W1, wu1)
        LLMR_PIPE_ITER(1, X1, X0, W1, W0, wu0)
        LLMR_PIPE_ITER(2, X2, X1, W0, W1, wu1)
        LLMR_PIPE_ITER(3, X0, X2, W1, W0, wu0)
        LLMR_PIPE_ITER(4, X1, X0, W0, W1, wu1)
        LLMR_PIPE_ITER(5, X2, X1, W1, W0, wu0)
    }
#undef LLMR_PIPE_ITER
    LLMR_WAIT_VMCNT(0);  // no DMA may still be writing this workgroup's LDS when it exits

    const bool vec_ok = (N % 4u) == 0u;
#pragma unroll
    for (int a = 0; a < TN; a++)
#pragma unroll
        for (int b = 0; b < TM; b++) {
            const uint32_t m = m0 + wm * WM + b * 32 + l32;
            if (m >= M) continue;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t n = n0 + wn * WN + a * 32 + 8 * g + 4 * kh;
                float* yp = Y + (uint64_t)m * N + n;
                const f32x4 v = {acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                                 acc[a][b][4 * g + 3]};
                if (vec_ok && n + 3 < N) {
                    *(f32x4*)yp = v;
                } else {
                    if (n < N) yp[0] = v.x;
                    if (n + 1 < N) yp[1] = v.y;
                    if (n + 2 < N) yp[2] = v.z;
                    if (n + 3 < N) yp[3] = v.w;
                }
            }
        }
}

// Generic path for shapes the tiled kernel does not take (Q8_0 with
// K % 64 == 32): one thread per output, operands and order as the MFMA path
// (fp16 activations, fp16 weight operands, f32 accumulation).
template <uint32_t WT, uint32_t XT>
__global__ void __launch_bounds__(256) gemm_q_generic(const uint8_t* __restrict__ W,
                                                      const void* __restrict__ X,
                                                      float* __restrict__ Y, uint32_t N,
                                                      uint32_t K, uint32_t M, uint32_t row_offset) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)M * N) return;
    const uint32_t m = (uint32_t)(gid / N), n = (uint32_t)(gid % N);
    const uint64_t row_bytes = (WT == kGgmlQ8_0) ? (uint64_t)(K / 32) * 34 : (uint64_t)(K / 256) * 144;
    const uint8_t* wr = W + (uint64_t)(row_offset + n) * row_bytes;
    float acc = 0.0f;
    for (uint32_t k = 0; k < K; k++) {
        float xv;
        if (XT == kGgmlF32)
            xv = ((const float*)X)[(uint64_t)m * K + k];
        else if (XT == kGgmlF16)
            xv = (float)((const _Float16*)X)[(uint64_t)m * K + k];
        else
            xv = __uint_as_float((uint32_t)((const uint16_t*)X)[(uint64_t)m * K + k] << 16);
        const float a = (float)(_Float16)xv;
        float b;
        if (WT == kGgmlQ8_0) {
            const uint8_t* blk = wr + (uint64_t)(k / 32) * 34;
            const _Float16 d = (_Float16)f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            b = (float)(_Float16)(d * (_Float16)(float)(int8_t)blk[2 + k % 32]);
        } else {
            const uint8_t* blk = wr + (uint64_t)(k / 256) * 144;
            const uint32_t e = k % 256, j = e >> 6, h = (e >> 5) & 1u, l = e & 31u;
            const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            const float dmin = f16_bits_to_f32((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
            uint32_t sc, mn;
            q4k_scale_min(2 * j + h, *(const uint32_t*)(blk + 4), *(const uint32_t*)(blk + 8),
                          *(const uint32_t*)(blk + 12), sc, mn);
            const uint32_t qb = blk[16 + j * 32 + l];
            const uint32_t q = h ? (qb >> 4) : (qb & 0xfu);
            b = (float)(_Float16)((d * (float)sc) * (float)q - dmin * (float)mn);
        }
        acc += a * b;
    }
    Y[(uint64_t)m * N + n] = acc;
}

template <uint32_t WT, uint32_t XT, int BM, int BN>
hipError_t launch_tiled(const void* w, const void* x, float* y, uint32_t N, uint32_t K, uint32_t M,
                        uint32_t row_offset, hipStream_t st) {
    constexpr uint32_t lds = 2u * (BM + BN) * kBK * 2;
    auto kern = gemm_q_mfma<WT, XT, BM, BN>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(256), lds, st, (const uint8_t*)w, x, y, N,
                       K, M, row_offset, tiles_m, tiles_n);
    return hipGetLastError();
}

template <uint32_t WT, uint32_t XT>
hipError_t dispatch_x(const void* w, const void* x, float* y, uint32_t N, uint32_t K, uint32_t M,
                      uint32_t row_offset, int num_cus, hipStream_t st) {
    if (WT == kGgmlQ8_0 && (K % kBK) != 0) {
        const uint64_t threads = (uint64_t)M * N;
        hipLaunchKernelGGL((gemm_q_generic<WT, XT>), dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0,
                           st, (const uint8_t*)w, x, y, N, K, M, row_offset);
        return hipGetLastError();
    }
    // Largest tile that still gives every CU at least ~1.5 workgroups.
    auto wgs = [&](uint32_t bm, uint32_t bn) {
        return (uint64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    };
    const uint64_t want = (uint64_t)num_cus * 3 / 2;
    if (wgs(256, 256) >= want) {
        // the pipelined kernel addresses activations and weight rows through
        // 32-bit buffer offsets: it needs the whole X and the used weight rows
        // to span less than 2 GiB
        const uint64_t rb = (WT == kGgmlQ8_0) ? (uint64_t)(K / 32) * 34 : (uint64_t)(K / 256) * 144;
        const bool fits31 = (uint64_t)M * K * 2u < (1ull << 31) && (uint64_t)N * rb < (1ull << 31);
        if constexpr (XT == kGgmlF32) {
            return launch_tiled<WT, XT, 256, 256>(w, x, y, N, K, M, row_offset, st);
        } else {
            if (!fits31) return launch_tiled<WT, XT, 256, 256>(w, x, y, N, K, M, row_offset, st);
            const uint32_t tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
            hipLaunchKernelGGL((gemm_q_pipe<WT, XT>), dim3(tiles_m * tiles_n), dim3(512), 0, st,
                               (const uint8_t*)w, x, y, N, K, M, row_offset, tiles_m, tiles_n);
            return hipGetLastError();
        }
    }
    if (wgs(128, 128) >= want) return launch_tiled<WT, XT, 128, 128>(w, x, y, N, K, M, row_offset, st);
    return launch_tiled<WT, XT, 64, 64>(w, x, y, N, K, M, row_offset, st);
}

template <uint32_t WT>
hipError_t dispatch_w(const void* w, uint32_t xtype, const void* x, float* y, uint32_t N, uint32_t K,
                      uint32_t M, uint32_t row_offset, int num_cus, hipStream_t st) {
    switch (xtype) {
        case kGgmlF32: return dispatch_x<WT, kGgmlF32>(w, x, y, N, K, M, row_offset, num_cus, st);
        case kGgmlF16: return dispatch_x<WT, kGgmlF16>(w, x, y, N, K, M, row_offset, num_cus, st);
        default: return dispatch_x<WT, kGgmlBF16>(w, x, y, N, K, M, row_offset, num_cus, st);
    }
}

}  // namespace

hipError_t launch_batch_matmul(const void* w, uint32_t wtype, const void* x, uint32_t xtype,
                               float* y, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                               uint32_t row_offset, int num_cus, hipStream_t st) {
    if (seq_len == 0 || out_dim == 0) return hipSuccess;
    if (wtype == kGgmlQ8_0)
        return dispatch_w<kGgmlQ8_0>(w, xtype, x, y, out_dim, in_dim, seq_len, row_offset, num_cus, st);
    return dispatch_w<kGgmlQ4K>(w, xtype, x, y, out_dim, in_dim, seq_len, row_offset, num_cus, st);
}

}  // namespace llmr
