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
#include <algorithm>
#include <type_traits>

#include "gemm_q_common.h"
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

template <uint32_t XT>
struct XLoad;

// bf16 / f16 activations: one 16-byte load per LDS chunk.
template <>
struct XLoad<kGgmlBF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const void* x, uint64_t elem, bool ok) {
        v = ok ? *(const u32x4*)((const uint16_t*)x + elem) : u32x4{0, 0, 0, 0};
    }
    // bf16 activations are used as bf16 operands (bf16 MFMA)
    template <uint32_t OT>
    __device__ __forceinline__ u32x4 to_op() const { return v; }
};
template <>
struct XLoad<kGgmlF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const void* x, uint64_t elem, bool ok) {
        v = ok ? *(const u32x4*)((const uint16_t*)x + elem) : u32x4{0, 0, 0, 0};
    }
    template <uint32_t OT>
    __device__ __forceinline__ u32x4 to_op() const { return v; }
};
// f32 activations: two 16-byte loads per LDS chunk, rounded to the operand
// type: fp16 as the reference's float16_t(v) (llm.slang:1673) against Q8_0,
// bf16 against Q4_K (its f32 range kept), both to nearest even.
template <>
struct XLoad<kGgmlF32> {
    f32x4 a, b;
    __device__ __forceinline__ void load(const void* x, uint64_t elem, bool ok) {
        const float* p = (const float*)x + elem;
        a = ok ? *(const f32x4*)p : f32x4{0, 0, 0, 0};
        b = ok ? *(const f32x4*)(p + 4) : f32x4{0, 0, 0, 0};
    }
    template <uint32_t OT>
    __device__ __forceinline__ u32x4 to_op() const {
        if constexpr (OT == kGgmlBF16)
            return u32x4{pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y),
                         pack_bf16x2(b.z, b.w)};
        else
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
    // bf16 operands: RN_bf16(d*q) (the product is exact in f32).
    template <uint32_t OT>
    __device__ __forceinline__ void store(uint8_t* lds, uint32_t r, uint32_t unit) const {
        (void)unit;
        const uint32_t wd[17] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x,
                                 c.y, c.z, c.w, d.x, d.y, d.z, d.w, e};
        if constexpr (OT == kGgmlBF16) {
            typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
            auto chunk = [](uint32_t q0, uint32_t q1, float dd) {
                bf16x8_t v;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[i] = (__bf16)(dd * (float)(int8_t)(q0 >> (8 * i)));
                    v[4 + i] = (__bf16)(dd * (float)(int8_t)(q1 >> (8 * i)));
                }
                return __builtin_bit_cast(u32x4, v);
            };
            const float d0 = f16_bits_to_f32(wd[0] & 0xffffu), d1 = f16_bits_to_f32(wd[8] >> 16);
#pragma unroll
            for (int ch = 0; ch < 4; ch++) {
                const uint32_t q0 = __builtin_amdgcn_alignbyte(wd[2 * ch + 1], wd[2 * ch], 2);
                const uint32_t q1 = __builtin_amdgcn_alignbyte(wd[2 * ch + 2], wd[2 * ch + 1], 2);
                *(u32x4*)(lds + lds_off(r, ch)) = chunk(q0, q1, d0);
                *(u32x4*)(lds + lds_off(r, 4 + ch)) = chunk(wd[9 + 2 * ch], wd[10 + 2 * ch], d1);
            }
            return;
        }
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
    // operands RN(d*sc*q - dmin*mn) of type OT (fp16 or bf16)
    template <uint32_t OT>
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
            if constexpr (OT == kGgmlBF16) {
                lo[2 * i] = q4_pair_bf16(l4, 0x04010400u, dsc0, dmn0);
                lo[2 * i + 1] = q4_pair_bf16(l4, 0x04030402u, dsc0, dmn0);
                hi[2 * i] = q4_pair_bf16(h4, 0x04010400u, dsc1, dmn1);
                hi[2 * i + 1] = q4_pair_bf16(h4, 0x04030402u, dsc1, dmn1);
            } else {
                lo[2 * i] = q4_pair(l4, 0x04010400u, dsc0, dmn0);
                lo[2 * i + 1] = q4_pair(l4, 0x04030402u, dsc0, dmn0);
                hi[2 * i] = q4_pair(h4, 0x04010400u, dsc1, dmn1);
                hi[2 * i + 1] = q4_pair(h4, 0x04030402u, dsc1, dmn1);
            }
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
            uint32_t tiles_n, uint32_t split_stages, uint64_t split_stride) {
    // MFMA operand type: bf16 for bf16 activations and for f32 ones against
    // Q4_K (batch_matmul_q4k keeps x in f32, so its range is kept), fp16
    // otherwise (the reference's float16_t(x) of batch_matmul_q8)
    constexpr uint32_t OT = (XT == kGgmlBF16 || (XT == kGgmlF32 && WT == kGgmlQ4K)) ? kGgmlBF16 : kGgmlF16;
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
    // split-K: workgroup row blockIdx.y takes stages [s_begin, s_end) and
    // writes its partial tile split_stride floats further on (one split: the
    // whole K, straight into Y)
    const uint32_t s_begin = blockIdx.y * split_stages;
    const uint32_t s_end = min(K / (uint32_t)kBK, s_begin + split_stages);
    Y += blockIdx.y * split_stride;

    // 64 x 64 tiles keep two register sets: the loads of stage s + 2 are in
    // flight while stage s is multiplied and stage s + 1 (landed) goes to LDS
    XLoad<XT> xa[X_PER_T], xb[X_PER_T];
    WLoad<WT> wa[W_PER_T], wb[W_PER_T];

    auto load_stage = [&](XLoad<XT>(&xl)[X_PER_T], WLoad<WT>(&wl)[W_PER_T], uint32_t s) {
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
    auto store_stage = [&](const XLoad<XT>(&xl)[X_PER_T], const WLoad<WT>(&wl)[W_PER_T], uint32_t s,
                           uint32_t buf) {
        uint8_t* As = smem + buf * STAGE;
        uint8_t* Bs = As + A_BYTES;
#pragma unroll
        for (int i = 0; i < X_PER_T; i++) {
            const uint32_t r = (tid >> 3) + 32u * i, c = tid & 7u;
            *(u32x4*)(As + lds_off(r, c)) = xl[i].template to_op<OT>();
        }
#pragma unroll
        for (int i = 0; i < W_PER_T; i++) {
            const uint32_t u = tid + 256u * i;
            if (u < (uint32_t)W_UNITS) {
                const uint32_t r = u / WLoad<WT>::kUnitsPerRow, unit = u % WLoad<WT>::kUnitsPerRow;
                if constexpr (WT == kGgmlQ4K)
                    wl[i].template store<OT>(Bs, r, unit, s * kBK);
                else
                    wl[i].template store<OT>(Bs, r, unit);
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

    auto compute_stage = [&](uint32_t buf) {
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
                        acc[a][b] = mfma16<OT>(wf[a], xf[b], acc[a][b]);
            }
        }
    };

    load_stage(xa, wa, s_begin);
    store_stage(xa, wa, s_begin, 0);
    if constexpr (BM * BN > 64 * 64) {
        // larger tiles: one stage of loads in flight (a second register set
        // would spill)
        __syncthreads();
        for (uint32_t s = s_begin; s < s_end; s++) {
            const uint32_t buf = (s - s_begin) & 1u;
            if (s + 1 < s_end) load_stage(xa, wa, s + 1);
            compute_stage(buf);
            if (s + 1 < s_end) store_stage(xa, wa, s + 1, buf ^ 1u);
            __syncthreads();
        }
    } else {
    if (s_begin + 1 < s_end) load_stage(xa, wa, s_begin + 1);
    __syncthreads();

    for (uint32_t s = s_begin; s < s_end; s += 2) {
        // stage s in LDS slot 0, stage s + 1 in registers xa / wa
        if (s + 2 < s_end) load_stage(xb, wb, s + 2);
        compute_stage(0);
        if (s + 1 < s_end) store_stage(xa, wa, s + 1, 1);
        __syncthreads();
        if (s + 1 >= s_end) break;
        // stage s + 1 in LDS slot 1, stage s + 2 in registers xb / wb
        if (s + 3 < s_end) load_stage(xa, wa, s + 3);
        compute_stage(1);
        if (s + 2 < s_end) store_stage(xb, wb, s + 2, 0);
        __syncthreads();
    }
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
// Persistent 256 x 256 tile kernel for 16-bit activations (gfx950).
//
// One workgroup per CU (grid = min(tiles, CUs)), 256 threads = one wave64
// per SIMD, each wave a 128 (tokens) x 128 (features) sub-tile held in 16
// v_mfma_f32_32x32x16 accumulators. A workgroup walks its tiles as one
// continuous sequence of K stages (64 wide), so the loads of the next tile
// start while the last stages of the current one are multiplied:
//  * activations go HBM -> LDS by buffer_load ... lds (16 B per lane) into a
//    3-slot ring, two stages ahead; each lane's source offset is permuted so
//    the fixed lane*16 LDS placement realizes the bank swizzle;
//  * each thread owns one weight row of the tile: its packed bytes for stage
//    s+2 are fetched into registers, dequantized during stage s into a
//    2-slot LDS ring (operand type = activation type);
//  * per stage: fragment reads are double-buffered in registers across the
//    four 16-wide k steps, and the one barrier sits after the third k step:
//    the MFMAs of the fourth step run after it, covering the barrier wait;
//  * a tile's f32 results are stored straight from the accumulators at the
//    first stage of the next tile, right after that stage's loads went out.
// Every row index lives in the per-lane buffer offset (rows past M or N read
// as zero through the descriptor size); stages past K (the count is padded
// to a multiple of 6 so the six ring-slot combinations are compile-time) and
// tiles past the workgroup's last read through a zero-size descriptor.
// ---------------------------------------------------------------------------

// SW (SwiGLU, batch_matmul_swiglu_q8, llm.slang:1769-1911): W holds the gate
// rows and W2 the up rows (N each, row_offset unused); a tile covers 128
// output features, whose 128 gate and 128 up rows form its 256 weight rows
// arranged so that each wave's 128 feature columns are 64 gate features
// followed by the same 64 up features: the epilogue writes
// silu(gate) * up from two accumulators of the same lane.
template <uint32_t WT, uint32_t XT, bool SW, uint32_t EPI = kEpiStore, bool GROUPED = false>
__global__ void __launch_bounds__(256, 1) gemm_q_persist(const PersistArgs args) {
    static_assert(!(SW && GROUPED) && (!SW || EPI == kEpiStore), "SwiGLU launches are single, plain stores");
    // every argument the kernel uses as a scalar local (the lambdas below
    // capture these, never the argument struct, which would otherwise be
    // addressed through private memory)
    const uint32_t N = args.N, K = args.K, tiles_m = args.tiles_m, tiles_n = args.tiles_n;
    const uint32_t ldy = args.ldy, ldy2 = args.ldy2, split = args.split, y2_bf16 = args.y2_bf16;
    const uint8_t* const W2 = args.W2;
    const uint8_t* const Wp0 = args.p[0].W;
    const uint8_t* const Wp1 = GROUPED ? args.p[1].W : nullptr;
    const void* const Xp0 = args.p[0].X;
    const void* const Xp1 = GROUPED ? args.p[1].X : nullptr;
    float* const Yp0 = args.p[0].Y;
    float* const Yp1 = GROUPED ? args.p[1].Y : nullptr;
    const float* const Gp0 = args.p[0].gate;
    const float* const Gp1 = GROUPED ? args.p[1].gate : nullptr;
    void* const Y2p0 = args.p[0].Y2;
    void* const Y2p1 = GROUPED ? args.p[1].Y2 : nullptr;
    const uint32_t Mp0 = args.p[0].M, Mp1 = GROUPED ? args.p[1].M : 0u;
    const uint32_t Rp0 = args.p[0].row_offset, Rp1 = GROUPED ? args.p[1].row_offset : 0u;
    const uint32_t Tp0 = args.p[0].tiles_m;
    static_assert(XT == kGgmlF16 || XT == kGgmlBF16, "16-bit activations only");
    constexpr uint32_t NT = SW ? 128u : 256u;  // output features per tile
    constexpr uint32_t TILE = 256u * 128u;  // bytes of one 256-row x 64-wide 16-bit tile
    constexpr int X_DMAS = 8;               // 1 KiB activation DMAs per wave per stage
    constexpr int W_LOADS = WRow<WT, XT>::kLoads;
    constexpr int IN_FLIGHT = X_DMAS + W_LOADS;  // one stage's loads
    __shared__ __attribute__((aligned(16))) uint8_t X0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t X1[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t X2[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t W0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t W1[TILE];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const uint32_t wm = wave & 1u, wn = wave >> 1;

    const uint32_t G = gridDim.x, total = tiles_m * tiles_n;
    const uint32_t n_tiles = (total - blockIdx.x + G - 1) / G;  // >= 1: grid <= total
    const uint32_t S = K / kBK;
    const uint32_t SP = (S + 5u) / 6u * 6u;
    const uint32_t rb = (WT == kGgmlQ8_0) ? (K / 32u) * 34u : (K / 256u) * 144u;
    const uint32_t xrow = K * 2u;

    // per-lane offsets (tile independent)
    // activation DMA i of wave w: rows 64w + 8i + lane/8, physical chunk lane%8,
    // logical chunk (lane%8) ^ lds_swz(row)
    uint32_t xvoff[X_DMAS];
#pragma unroll
    for (int i = 0; i < X_DMAS; i++) {
        const uint32_t row = 64u * wave + 8u * i + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ lds_swz(row);
        xvoff[i] = row * xrow + c * 16u;
    }
    // Thread tid loads one weight row of the tile. SW: waves 0-1 the gate rows
    // 0..127 and waves 2-3 the up rows 0..127 of the tile's features (one
    // descriptor per wave), placed at LDS rows gate 0-63 | up 0-63 | gate
    // 64-127 | up 64-127 (waves 1 and 2 swap places).
    const uint32_t wvoff = (SW ? (tid & 127u) : tid) * rb;
    const uint32_t wrow = SW ? (wave == 1u ? tid + 64u : wave == 2u ? tid - 64u : tid) : tid;
    const uint32_t wbase = wrow * 128u + (lds_swz(wrow) << 4);  // its LDS chunk 0
    // fragment offsets per 16-wide k step t: chunk 4(t>>1) + 2kh + (t&1) of
    // rows (block) + l32; the swizzle term depends only on l32
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t ch = 4u * (t >> 1) + 2u * kh + (t & 1);
        xoff[t] = lds_off(wm * 128u + l32, ch);
        woff[t] = lds_off(wn * 128u + l32, ch);
    }

    // Load side. Activations are fetched two stages ahead, weights three
    // (their row-strided reads have the longer latency); each stream walks
    // the workgroup's (tile, stage) sequence with its own cursor.
    struct Cursor {
        uint32_t s;               // stage within the tile
        const uint8_t* base;      // the tile's first activation row / weight row
        uint32_t size;            // bytes of valid rows from base (0 past the last tile)
    };
    // tile k of this workgroup: its problem, its first row in that problem,
    // its first output feature
    auto tile_origin = [&](uint32_t k, uint32_t& p, uint32_t& m0, uint32_t& n0) {
        uint32_t tm, tn;
        map_tile_persist(blockIdx.x + k * G, G, tiles_m, tiles_n, tm, tn);
        p = GROUPED && tm >= Tp0 ? 1u : 0u;
        m0 = (tm - (p ? Tp0 : 0u)) * 256u;
        n0 = tn * NT;
    };
    auto x_tile = [&](Cursor& c, uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        c.s = 0;
        c.base = (const uint8_t*)pick(p, Xp0, Xp1) + (uint64_t)m0 * xrow;
        c.size = k < n_tiles ? (pick(p, Mp0, Mp1) - m0) * xrow : 0u;
    };
    auto w_tile = [&](Cursor& c, uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        c.s = 0;
        if constexpr (SW)
            c.base = (wave < 2u ? Wp0 : W2) + (uint64_t)n0 * rb;
        else
            c.base = pick(p, Wp0, Wp1) + (uint64_t)(pick(p, Rp0, Rp1) + n0) * rb;
        c.size = k < n_tiles ? (N - n0) * rb : 0u;
    };
    Cursor cx{0, nullptr, 0}, cw{0, nullptr, 0};
    // the tile after the one being multiplied, prepared once per tile: a
    // cursor moving on to it only copies it (no per-stage tile arithmetic;
    // a tile has at least 6 stages, more than the loads run ahead)
    Cursor nx{0, nullptr, 0}, nw{0, nullptr, 0};
    auto advance = [&](Cursor& c, const Cursor& next) {
        if (++c.s == SP) c = next;
    };
    // one activation DMA (1 KiB: rows 64w + 8i .. +7 of the slot) of stage `so`/128
    auto dma = [&](rsrc_t xr, uint8_t* Xs, int i, uint32_t so) {
        uint8_t* dst = Xs + wave * (64u * 128u) + 1024u * i;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)dst, 16, xvoff[i], so, 0, 0);
    };
    WRow<WT, XT> R0, R1, R2;
    // whole-stage loads (prologue): weights of the W cursor's stage into U,
    // activations of the X cursor's stage into slot Xs
    auto issue_w_all = [&](WRow<WT, XT>& U) {
        const rsrc_t wr = make_rsrc(cw.base, cw.s < S ? cw.size : 0u);
        static_for<0, W_LOADS>([&](auto L) { U.template load<decltype(L)::value>(wr, wvoff, cw.s); });
        advance(cw, nw);
    };
    auto issue_x_all = [&](uint8_t* Xs) {
        const rsrc_t xr = make_rsrc(cx.base, cx.s < S ? cx.size : 0u);
#pragma unroll
        for (int i = 0; i < X_DMAS; i++) dma(xr, Xs, i, cx.s * 128u);
        advance(cx, nx);
    };
    // A stage's loads in issue order: the W_LOADS weight loads of W(g+3),
    // then the X_DMAS activation DMAs of X(g+2); part p of 4 issues the
    // slice [p n / 4, (p+1) n / 4) of that list.
    constexpr int N_OPS = W_LOADS + X_DMAS;
    auto issue_part = [&](auto PART, rsrc_t wr, uint32_t ws, rsrc_t xr, uint32_t xso, uint8_t* Xs,
                          WRow<WT, XT>& U) {
        constexpr int p = decltype(PART)::value;
        static_for<p * N_OPS / 4, (p + 1) * N_OPS / 4>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if constexpr (i < W_LOADS)
                U.template load<i>(wr, wvoff, ws);
            else
                dma(xr, Xs, i - W_LOADS, xso);
        });
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f32x16{};

    auto read_frags = [&](Frags& f, const uint8_t* Xs, const uint8_t* Ws, int t) {
#pragma unroll
        for (int b = 0; b < 4; b++) f.x[b] = *(const f16x8*)(Xs + b * 32 * 128 + xoff[t]);
#pragma unroll
        for (int a = 0; a < 4; a++) f.w[a] = *(const f16x8*)(Ws + a * 32 * 128 + woff[t]);
    };
    auto mfma_step = [&](const Frags& f) {
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) acc[a][b] = mfma16<XT>(f.w[a], f.x[b], acc[a][b]);
    };
    // Store the accumulators as tile k's results and clear them (N % 4 == 0,
    // host-checked: a lane's four consecutive features are all in range or
    // all out).
    auto store_tile = [&](uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        store_tile_256<SW, EPI>(acc, pick(p, Yp0, Yp1), pick(p, Gp0, Gp1), pick(p, Y2p0, Y2p1), pick(p, Mp0, Mp1), N,
                                m0, n0, wm, wn, l32, kh, ldy, ldy2, split, y2_bf16);
    };

    // prologue, issued in the steady state's order (a stage issues the
    // weights of g+3, then the activations of g+2): W0 | W1 X0 | W2 X1; then
    // stage 0's weights are dequantized and its activations have landed
    x_tile(cx, 0);
    w_tile(cw, 0);
    x_tile(nx, 1);
    w_tile(nw, 1);
    issue_w_all(R0);
    issue_w_all(R1);
    issue_x_all(X0);
    issue_w_all(R2);
    issue_x_all(X1);
    LLMR_WAIT_VMCNT(2 * W_LOADS + 2 * X_DMAS);
    {
        const auto sc0 = R0.scale(0);
        R0.template store<0>(W0, sc0, wbase);
        R0.template store<1>(W0, sc0, wbase);
        R0.template store<2>(W0, sc0, wbase);
        R0.template store<3>(W0, sc0, wbase);
    }
    LLMR_STAGE_BARRIER(IN_FLIGHT);

    Frags F0, F1;

    // Global stage g: slots X[g%3], W[g%2]; W(g+1) is in register row R[(g+1)%3].
    //   wait for W(g+1) (issued first two stages ago: the activation DMAs of
    //   that stage and all of last stage's loads may stay in flight);
    //   k step A: MFMA (g-1,3), frags (g,0), dequant part 0, loads part 0
    //   k step B: MFMA (g,0), frags (g,1), dequant part 1, loads part 1
    //   k step C: MFMA (g,1), frags (g,2), dequant part 2, loads part 2
    //   k step D: MFMA (g,2), frags (g,3), dequant part 3, loads part 3
    //   (loads: weights of g+3 -> R[g%3], then activations of g+2 -> X[(g+2)%3]);
    //   barrier once X(g+1) has landed (issued last in the previous stage:
    //   this stage's loads may stay in flight) and the LDS writes are done.
    // Loads run ahead across tile boundaries (each stream walks the
    // workgroup's tiles on its own), so a tile's first stages are already in
    // flight when its predecessor's results are stored.
#define LLMR_PERSIST_STAGE(XC, WC, XD, WNX, RN, RL, NEXT)                                    \
    {                                                                                       \
        const rsrc_t wr_ = make_rsrc(cw.base, cw.s < S ? cw.size : 0u);                      \
        const rsrc_t xr_ = make_rsrc(cx.base, cx.s < S ? cx.size : 0u);                      \
        const uint32_t ws_ = cw.s, xso_ = cx.s * 128u;                                      \
        LLMR_WAIT_VMCNT(X_DMAS + IN_FLIGHT);                                                \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        const auto sc_ = RN.scale(NEXT);                                                    \
        issue_part(std::integral_constant<int, 0>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F0, XC, WC, 0);                                                          \
        mfma_step(F1);                                                                      \
        RN.template store<0>(WNX, sc_, wbase);                                              \
        LLMR_STEP_SCHEDULE_A;                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 1>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F1, XC, WC, 1);                                                          \
        mfma_step(F0);                                                                      \
        RN.template store<1>(WNX, sc_, wbase);                                              \
        LLMR_STEP_SCHEDULE;                                                                 \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 2>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F0, XC, WC, 2);                                                          \
        mfma_step(F1);                                                                      \
        RN.template store<2>(WNX, sc_, wbase);                                              \
        LLMR_STEP_SCHEDULE;                                                                 \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 3>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F1, XC, WC, 3);                                                          \
        mfma_step(F0);                                                                      \
        RN.template store<3>(WNX, sc_, wbase);                                              \
        LLMR_STEP_SCHEDULE;                                                                 \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        advance(cw, nw);                                                                    \
        advance(cx, nx);                                                                    \
        LLMR_STAGE_BARRIER(IN_FLIGHT);                                                      \
    }
    for (uint32_t k = 0; k < n_tiles; k++) {
        if (k > 0) {  // the load cursors have moved on to tile k: prepare tile k+1
            x_tile(nx, k + 1);
            w_tile(nw, k + 1);
        }
        // the first stage's "previous step" multiplies nothing
#pragma unroll
        for (int i = 0; i < 4; i++) {
            F1.x[i] = f16x8{};
            F1.w[i] = f16x8{};
        }
        for (uint32_t s0 = 0; s0 < SP; s0 += 6) {
            LLMR_PERSIST_STAGE(X0, W0, X2, W1, R1, R0, s0 + 1)
            LLMR_PERSIST_STAGE(X1, W1, X0, W0, R2, R1, s0 + 2)
            LLMR_PERSIST_STAGE(X2, W0, X1, W1, R0, R2, s0 + 3)
            LLMR_PERSIST_STAGE(X0, W1, X2, W0, R1, R0, s0 + 4)
            LLMR_PERSIST_STAGE(X1, W0, X0, W1, R2, R1, s0 + 5)
            LLMR_PERSIST_STAGE(X2, W1, X1, W0, R0, R2, s0 + 6 == SP ? 0u : s0 + 6)
        }
        mfma_step(F1);
        store_tile(k);
    }
#undef LLMR_PERSIST_STAGE
    LLMR_WAIT_VMCNT(0);  // no DMA may still be writing this workgroup's LDS when it exits
}

// ---------------------------------------------------------------------------
// gemm_q_persist8: the persistent kernel on 8 waves (two per SIMD). A wave's
// VALU and LDS instructions issue between its own MFMAs only at a cost
// (about 2 cycles per VALU instruction on top of the MFMA's 32), but they
// are free while the other wave of the SIMD keeps the matrix core busy; and
// one wave alone reads LDS at ~32 B/clk, eight waves at ~220 B/clk. The
// tile stays 256 x 256 with the same LDS rings, stage order and barriers;
// wave w owns tokens 128 (w & 1) .. +127 x features 64 ((w >> 1) & 3) .. +63
// (2 x 4 accumulators of 32 x 32), and two threads share each weight row.
// ---------------------------------------------------------------------------

// Half a weight row's stage for the 8-wave kernel: half h (uniform in a
// wave) dequantizes the LDS chunks 2h, 2h+1, 4+2h, 4+2h+1 of the row (Q4_K:
// qs bytes 16h .. 16h+15 of the stage's 32, low and high nibbles) or chunks
// 4h .. 4h+3 (Q8_0: block h of the stage's two). Part p of 4 writes one chunk.
template <uint32_t WT, uint32_t OT>
struct WHalf;

template <uint32_t OT>
struct WHalf<kGgmlQ4K, OT> {
    static constexpr int kLoads = 2;
    u32x4 hdr, q;
    template <int L>
    __device__ __forceinline__ void load(rsrc_t r, uint32_t voff, uint32_t s, uint32_t h) {
        const uint32_t sh = (s >> 2) * 144u;
        if constexpr (L == 0) hdr = bload16(r, voff, sh);
        if constexpr (L == 1) q = bload16(r, voff, sh + 16u + 32u * (s & 3u) + 16u * h);
    }
    struct Scale {
        float s0, b0, s1, b1;
    };
    // the same operand RN(d*sc*q - dmin*mn) as WRow<kGgmlQ4K>
    __device__ __forceinline__ Scale scale(uint32_t s, uint32_t) const {
        const uint32_t j = s & 3u;
        const float d = f16_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(hdr.x >> 16);
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(2 * j, hdr.y, hdr.z, hdr.w, sc0, mn0);
        q4k_scale_min(2 * j + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
        return Scale{d * (float)sc0 * 16777216.0f, -(dmin * (float)mn0), d * (float)sc1 * 1048576.0f,
                     -(dmin * (float)mn1)};
    }
    template <int P>
    __device__ __forceinline__ void store(uint8_t* lds, const Scale& c, uint32_t base, uint32_t h) const {
        constexpr bool HI = (P & 1) != 0;
        const uint32_t w0 = P < 2 ? q.x : q.z, w1 = P < 2 ? q.y : q.w;
        const uint32_t mask = HI ? 0xf0f0f0f0u : 0x0f0f0f0fu;
        const uint32_t m0 = w0 & mask, m1 = w1 & mask;
        const float s = HI ? c.s1 : c.s0, b = HI ? c.b1 : c.b0;
        const u32x4 v = {fma_pair<OT>(sub16x2(m0, kSelLo), s, b), fma_pair<OT>(sub16x2(m0, kSelHi), s, b),
                         fma_pair<OT>(sub16x2(m1, kSelLo), s, b), fma_pair<OT>(sub16x2(m1, kSelHi), s, b)};
        const uint32_t ch = (HI ? 4u : 0u) + 2u * h + (uint32_t)(P >> 1);
        *(u32x4*)(lds + (base ^ (ch << 4))) = v;
    }
};

template <uint32_t OT>
struct WHalf<kGgmlQ8_0, OT> {
    static constexpr int kLoads = 3;
    u32x4 a, b;
    uint32_t e;
    // bytes [68 s + 32 h, +36): block h's scale is the half at byte 34 h - 32 h
    // (h = 0: low half of dword 0; h = 1: high half), its 32 quants start at
    // byte 2 (h = 0, unaligned) or 4 (h = 1)
    template <int L>
    __device__ __forceinline__ void load(rsrc_t r, uint32_t voff, uint32_t s, uint32_t h) {
        const uint32_t so = 68u * s + 32u * h;
        if constexpr (L == 0) a = bload16(r, voff, so);
        if constexpr (L == 1) b = bload16(r, voff + 16u, so);
        if constexpr (L == 2) e = bload4(r, voff + 32u, so);
    }
    struct Scale {
        float s, b;  // bf16: (2^24 d, -128 d); f16: (d, -)
    };
    __device__ __forceinline__ Scale scale(uint32_t, uint32_t h) const {
        const float d = f16_bits_to_f32(h ? a.x >> 16 : a.x & 0xffffu);
        if constexpr (OT == kGgmlBF16)
            return Scale{d * 16777216.0f, -128.0f * d};
        else
            return Scale{d, 0.0f};
    }
    __device__ __forceinline__ uint32_t word(int i) const {
        return i < 4 ? a[i] : i < 8 ? b[i - 4] : e;
    }
    template <int P>
    __device__ __forceinline__ void store(uint8_t* lds, const Scale& k, uint32_t base, uint32_t h) const {
        // quant dwords 2P, 2P+1 of the block
        const uint32_t q0 = h ? word(2 * P + 1) : __builtin_amdgcn_alignbyte(word(2 * P + 1), word(2 * P), 2);
        const uint32_t q1 = h ? word(2 * P + 2) : __builtin_amdgcn_alignbyte(word(2 * P + 2), word(2 * P + 1), 2);
        u32x4 v;
        if constexpr (OT == kGgmlBF16) {
            const uint32_t u0 = q0 ^ 0x80808080u, u1 = q1 ^ 0x80808080u;
            v = u32x4{fma_pair<OT>(sub16x2(u0, kSelLo), k.s, k.b), fma_pair<OT>(sub16x2(u0, kSelHi), k.s, k.b),
                      fma_pair<OT>(sub16x2(u1, kSelLo), k.s, k.b), fma_pair<OT>(sub16x2(u1, kSelHi), k.s, k.b)};
        } else {
            const _Float16 d = (_Float16)k.s;
            v = q8x8_f16(q0, q1, f16x2{d, d});
        }
        const uint32_t ch = 4u * h + (uint32_t)P;
        *(u32x4*)(lds + (base ^ (ch << 4))) = v;
    }
};

// One 16-wide k step of the 8-wave kernel: 8 MFMAs, the next step's six
// fragment reads after the first six, the dequantization's VALU, its LDS
// write and the step's loads in between.
#define LLMR8_SLOT_R LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x002, 2)
#define LLMR8_STEP_SCHEDULE                                                                 \
    LLMR8_SLOT_R; LLMR8_SLOT_R; LLMR8_SLOT_R; LLMR8_SLOT_R; LLMR8_SLOT_R; LLMR8_SLOT_R;     \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 4); LLMR_SGB(0x200, 1);                             \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x002, 4); LLMR_SGB(0x020, 2)

struct Frags8 {
    f16x8 x[4], w[2];
};

template <uint32_t WT, uint32_t XT, uint32_t EPI = kEpiStore, bool GROUPED = false>
__global__ void __launch_bounds__(512, 1) gemm_q_persist8(const PersistArgs args) {
    // every argument the kernel uses as a scalar local (see gemm_q_persist)
    const uint32_t N = args.N, K = args.K, tiles_m = args.tiles_m, tiles_n = args.tiles_n;
    const uint32_t ldy = args.ldy, ldy2 = args.ldy2, split = args.split, y2_bf16 = args.y2_bf16;
    const uint8_t* const Wp0 = args.p[0].W;
    const uint8_t* const Wp1 = GROUPED ? args.p[1].W : nullptr;
    const void* const Xp0 = args.p[0].X;
    const void* const Xp1 = GROUPED ? args.p[1].X : nullptr;
    float* const Yp0 = args.p[0].Y;
    float* const Yp1 = GROUPED ? args.p[1].Y : nullptr;
    const float* const Gp0 = args.p[0].gate;
    const float* const Gp1 = GROUPED ? args.p[1].gate : nullptr;
    void* const Y2p0 = args.p[0].Y2;
    void* const Y2p1 = GROUPED ? args.p[1].Y2 : nullptr;
    const uint32_t Mp0 = args.p[0].M, Mp1 = GROUPED ? args.p[1].M : 0u;
    const uint32_t Rp0 = args.p[0].row_offset, Rp1 = GROUPED ? args.p[1].row_offset : 0u;
    const uint32_t Tp0 = args.p[0].tiles_m;
    static_assert(XT == kGgmlF16 || XT == kGgmlBF16, "16-bit activations only");
    constexpr uint32_t TILE = 256u * 128u;  // bytes of one 256-row x 64-wide 16-bit tile
    constexpr int X_DMAS = 4;               // 1 KiB activation DMAs per wave per stage
    constexpr int W_LOADS = WHalf<WT, XT>::kLoads;
    constexpr int IN_FLIGHT = X_DMAS + W_LOADS;  // one stage's loads
    __shared__ __attribute__((aligned(16))) uint8_t X0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t X1[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t X2[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t W0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t W1[TILE];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const uint32_t wm = wave & 1u, wn = (wave >> 1) & 3u;
    const uint32_t wh = wave >> 2;  // the weight-row half this wave dequantizes

    const uint32_t G = gridDim.x, total = tiles_m * tiles_n;
    const uint32_t n_tiles = (total - blockIdx.x + G - 1) / G;  // >= 1: grid <= total
    const uint32_t S = K / kBK;
    const uint32_t SP = (S + 5u) / 6u * 6u;
    const uint32_t rb = (WT == kGgmlQ8_0) ? (K / 32u) * 34u : (K / 256u) * 144u;
    const uint32_t xrow = K * 2u;

    // activation DMA i of wave w: rows 32w + 8i + lane/8, physical chunk
    // lane%8, logical chunk (lane%8) ^ lds_swz(row)
    uint32_t xvoff[X_DMAS];
#pragma unroll
    for (int i = 0; i < X_DMAS; i++) {
        const uint32_t row = 32u * wave + 8u * i + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ lds_swz(row);
        xvoff[i] = row * xrow + c * 16u;
    }
    // thread tid dequantizes half wh of weight row tid % 256 of the tile
    const uint32_t wrow = tid & 255u;
    const uint32_t wvoff = wrow * rb;
    const uint32_t wbase = wrow * 128u + (lds_swz(wrow) << 4);  // its LDS chunk 0
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t ch = 4u * (t >> 1) + 2u * kh + (t & 1);
        xoff[t] = lds_off(wm * 128u + l32, ch);
        woff[t] = lds_off(wn * 64u + l32, ch);
    }

    struct Cursor {
        uint32_t s;
        const uint8_t* base;
        uint32_t size;
    };
    auto tile_origin = [&](uint32_t k, uint32_t& p, uint32_t& m0, uint32_t& n0) {
        uint32_t tm, tn;
        map_tile_persist(blockIdx.x + k * G, G, tiles_m, tiles_n, tm, tn);
        p = GROUPED && tm >= Tp0 ? 1u : 0u;
        m0 = (tm - (p ? Tp0 : 0u)) * 256u;
        n0 = tn * 256u;
    };
    auto x_tile = [&](Cursor& c, uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        c.s = 0;
        c.base = (const uint8_t*)pick(p, Xp0, Xp1) + (uint64_t)m0 * xrow;
        c.size = k < n_tiles ? (pick(p, Mp0, Mp1) - m0) * xrow : 0u;
    };
    auto w_tile = [&](Cursor& c, uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        c.s = 0;
        c.base = pick(p, Wp0, Wp1) + (uint64_t)(pick(p, Rp0, Rp1) + n0) * rb;
        c.size = k < n_tiles ? (N - n0) * rb : 0u;
    };
    Cursor cx{0, nullptr, 0}, cw{0, nullptr, 0};
    Cursor nx{0, nullptr, 0}, nw{0, nullptr, 0};
    auto advance = [&](Cursor& c, const Cursor& next) {
        if (++c.s == SP) c = next;
    };
    auto dma = [&](rsrc_t xr, uint8_t* Xs, int i, uint32_t so) {
        uint8_t* dst = Xs + wave * (32u * 128u) + 1024u * i;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)dst, 16, xvoff[i], so, 0, 0);
    };
    WHalf<WT, XT> R0, R1, R2;
    auto issue_w_all = [&](WHalf<WT, XT>& U) {
        const rsrc_t wr = make_rsrc(cw.base, cw.s < S ? cw.size : 0u);
        static_for<0, W_LOADS>([&](auto L) { U.template load<decltype(L)::value>(wr, wvoff, cw.s, wh); });
        advance(cw, nw);
    };
    auto issue_x_all = [&](uint8_t* Xs) {
        const rsrc_t xr = make_rsrc(cx.base, cx.s < S ? cx.size : 0u);
#pragma unroll
        for (int i = 0; i < X_DMAS; i++) dma(xr, Xs, i, cx.s * 128u);
        advance(cx, nx);
    };
    constexpr int N_OPS = W_LOADS + X_DMAS;
    auto issue_part = [&](auto PART, rsrc_t wr, uint32_t ws, rsrc_t xr, uint32_t xso, uint8_t* Xs,
                          WHalf<WT, XT>& U) {
        constexpr int p = decltype(PART)::value;
        static_for<p * N_OPS / 4, (p + 1) * N_OPS / 4>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if constexpr (i < W_LOADS)
                U.template load<i>(wr, wvoff, ws, wh);
            else
                dma(xr, Xs, i - W_LOADS, xso);
        });
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f32x16{};

    auto read_frags = [&](Frags8& f, const uint8_t* Xs, const uint8_t* Ws, int t) {
#pragma unroll
        for (int b = 0; b < 4; b++) f.x[b] = *(const f16x8*)(Xs + b * 32 * 128 + xoff[t]);
#pragma unroll
        for (int a = 0; a < 2; a++) f.w[a] = *(const f16x8*)(Ws + a * 32 * 128 + woff[t]);
    };
    auto mfma_step = [&](const Frags8& f) {
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) acc[a][b] = mfma16<XT>(f.w[a], f.x[b], acc[a][b]);
    };
    // Store the accumulators as tile k's results and clear them (N % 4 == 0,
    // host-checked). nw = n - 4 kh is uniform in the wave; with split % 8 ==
    // 0 (host-checked) nw < split is a uniform branch.
    auto store_tile = [&](uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        const uint32_t M = pick(p, Mp0, Mp1);
        float* const Y = pick(p, Yp0, Yp1);
        auto each = [&](auto&& f) __attribute__((always_inline)) {
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const uint32_t m = m0 + wm * 128u + b * 32u + l32;
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const uint32_t nw = n0 + wn * 64u + a * 32u + 8u * g;
                        const uint32_t n = nw + 4u * kh;
                        if (m < M && n < N)
                            f(m, n, nw, f32x4{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2],
                                              acc[a][b][4 * g + 3]});
                    }
                    acc[a][b] = f32x16{};
                }
        };
        if constexpr (EPI == kEpiResidual) {
            const float* const gate = pick(p, Gp0, Gp1);
            each([&](uint32_t m, uint32_t n, uint32_t, f32x4 v) __attribute__((always_inline)) {
                f32x4* const h = (f32x4*)(Y + (uint64_t)m * ldy + n);
                const f32x4 gv = gate ? *(const f32x4*)(gate + n) : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
                *h = *h + gv * v;
            });
        } else if constexpr (EPI == kEpiSplitGelu) {
            uint16_t* const Y2 = (uint16_t*)pick(p, Y2p0, Y2p1);
            const uint32_t bf = y2_bf16;
            each([&](uint32_t m, uint32_t n, uint32_t nw, f32x4 v) __attribute__((always_inline)) {
                if (nw < split) {
                    *(f32x4*)(Y + (uint64_t)m * ldy + n) = v;
                } else {
                    const f32x4 gl{gelu_tanh(v.x), gelu_tanh(v.y), gelu_tanh(v.z), gelu_tanh(v.w)};
                    u32x2 o;
                    if (bf) {
                        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
                        o.x = __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)gl.x, (__bf16)gl.y});
                        o.y = __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)gl.z, (__bf16)gl.w});
                    } else {
                        o = u32x2{pack_f16x2(gl.x, gl.y), pack_f16x2(gl.z, gl.w)};
                    }
                    *(u32x2*)(Y2 + (uint64_t)m * ldy2 + (n - split)) = o;
                }
            });
        } else {
            each([&](uint32_t m, uint32_t n, uint32_t, f32x4 v) __attribute__((always_inline)) {
                *(f32x4*)(Y + (uint64_t)m * ldy + n) = v;
            });
        }
    };

    // prologue, as gemm_q_persist's: W0 | W1 X0 | W2 X1, then stage 0's
    // weights are dequantized and its activations have landed
    x_tile(cx, 0);
    w_tile(cw, 0);
    x_tile(nx, 1);
    w_tile(nw, 1);
    issue_w_all(R0);
    issue_w_all(R1);
    issue_x_all(X0);
    issue_w_all(R2);
    issue_x_all(X1);
    LLMR_WAIT_VMCNT(2 * W_LOADS + 2 * X_DMAS);
    {
        const auto sc0 = R0.scale(0, wh);
        R0.template store<0>(W0, sc0, wbase, wh);
        R0.template store<1>(W0, sc0, wbase, wh);
        R0.template store<2>(W0, sc0, wbase, wh);
        R0.template store<3>(W0, sc0, wbase, wh);
    }
    LLMR_STAGE_BARRIER(IN_FLIGHT);

    Frags8 F0, F1;
    // the stage of gemm_q_persist with this kernel's fragments and schedule
#define LLMR_PERSIST8_STAGE(XC, WC, XD, WNX, RN, RL, NEXT)                                   \
    {                                                                                       \
        const rsrc_t wr_ = make_rsrc(cw.base, cw.s < S ? cw.size : 0u);                      \
        const rsrc_t xr_ = make_rsrc(cx.base, cx.s < S ? cx.size : 0u);                      \
        const uint32_t ws_ = cw.s, xso_ = cx.s * 128u;                                      \
        LLMR_WAIT_VMCNT(X_DMAS + IN_FLIGHT);                                                \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        const auto sc_ = RN.scale(NEXT, wh);                                                \
        issue_part(std::integral_constant<int, 0>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F0, XC, WC, 0);                                                          \
        mfma_step(F1);                                                                      \
        RN.template store<0>(WNX, sc_, wbase, wh);                                          \
        LLMR8_STEP_SCHEDULE;                                                                \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 1>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F1, XC, WC, 1);                                                          \
        mfma_step(F0);                                                                      \
        RN.template store<1>(WNX, sc_, wbase, wh);                                          \
        LLMR8_STEP_SCHEDULE;                                                                \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 2>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F0, XC, WC, 2);                                                          \
        mfma_step(F1);                                                                      \
        RN.template store<2>(WNX, sc_, wbase, wh);                                          \
        LLMR8_STEP_SCHEDULE;                                                                \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 3>{}, wr_, ws_, xr_, xso_, XD, RL);          \
        read_frags(F1, XC, WC, 3);                                                          \
        mfma_step(F0);                                                                      \
        RN.template store<3>(WNX, sc_, wbase, wh);                                          \
        LLMR8_STEP_SCHEDULE;                                                                \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        advance(cw, nw);                                                                    \
        advance(cx, nx);                                                                    \
        LLMR_STAGE_BARRIER(IN_FLIGHT);                                                      \
    }
    for (uint32_t k = 0; k < n_tiles; k++) {
        if (k > 0) {
            x_tile(nx, k + 1);
            w_tile(nw, k + 1);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) F1.x[i] = f16x8{};
#pragma unroll
        for (int i = 0; i < 2; i++) F1.w[i] = f16x8{};
        for (uint32_t s0 = 0; s0 < SP; s0 += 6) {
            LLMR_PERSIST8_STAGE(X0, W0, X2, W1, R1, R0, s0 + 1)
            LLMR_PERSIST8_STAGE(X1, W1, X0, W0, R2, R1, s0 + 2)
            LLMR_PERSIST8_STAGE(X2, W0, X1, W1, R0, R2, s0 + 3)
            LLMR_PERSIST8_STAGE(X0, W1, X2, W0, R1, R0, s0 + 4)
            LLMR_PERSIST8_STAGE(X1, W0, X0, W1, R2, R1, s0 + 5)
            LLMR_PERSIST8_STAGE(X2, W1, X1, W0, R0, R2, s0 + 6 == SP ? 0u : s0 + 6)
        }
        mfma_step(F1);
        store_tile(k);
    }
#undef LLMR_PERSIST8_STAGE
    LLMR_WAIT_VMCNT(0);  // no DMA may still be writing this workgroup's LDS when it exits
}

// Generic path for shapes the tiled kernel does not take (Q8_0 with
// K % 64 == 32): one thread per output, operands as the MFMA paths (bf16
// activations and weight operands for bf16 inputs, fp16 otherwise; f32
// accumulation).
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
        constexpr bool bf = XT == kGgmlBF16;
        const float a = bf ? xv : (float)(_Float16)xv;
        float b;
        if (WT == kGgmlQ8_0) {
            const uint8_t* blk = wr + (uint64_t)(k / 32) * 34;
            const float df = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            const _Float16 d = (_Float16)df;
            const float q = (float)(int8_t)blk[2 + k % 32];
            b = bf ? (float)(__bf16)(df * q) : (float)(_Float16)(d * (_Float16)q);
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
            const float v = __builtin_fmaf((float)q, d * (float)sc, -(dmin * (float)mn));
            b = bf ? (float)(__bf16)v : (float)(_Float16)v;
        }
        acc += a * b;
    }
    Y[(uint64_t)m * N + n] = acc;
}

// Y = sum over the split partials P[0 .. splits-1] (each `stride` floats),
// added in split order; four floats per thread.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ P, float* __restrict__ Y,
                                                            uint64_t n4, uint32_t splits, uint64_t stride) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n4) return;
    f32x4 a = ((const f32x4*)P)[i];
    for (uint32_t q = 1; q < splits; q++) a += ((const f32x4*)(P + q * stride))[i];
    ((f32x4*)Y)[i] = a;
}

}  // namespace

hipError_t launch_splitk_reduce(const float* part, float* y, uint64_t mn, uint32_t splits, hipStream_t st) {
    const uint64_t n4 = mn / 4;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((uint32_t)((n4 + 255) / 256)), dim3(256), 0, st, part, y, n4,
                       splits, mn);
    return hipGetLastError();
}

namespace {

// splits > 1: the partials go to `part` (splits * M * N floats), then the
// reduction writes Y.
template <uint32_t WT, uint32_t XT, int BM, int BN>
hipError_t launch_tiled(const void* w, const void* x, float* y, uint32_t N, uint32_t K, uint32_t M,
                        uint32_t row_offset, uint32_t splits, float* part, hipStream_t st) {
    constexpr uint32_t lds = 2u * (BM + BN) * kBK * 2;
    auto kern = gemm_q_mfma<WT, XT, BM, BN>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const uint32_t n_stages = K / kBK;
    // every split must own at least one stage: the kernel loads its first
    // stage unconditionally
    if (!plan::splits_nonempty(n_stages, splits) || (splits > 1 && (uint64_t)M * N % 4)) return hipErrorInvalidValue;
    const uint32_t per = (n_stages + splits - 1) / splits;
    const uint64_t mn = (uint64_t)M * N;
    hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n, splits), dim3(256), lds, st, (const uint8_t*)w, x,
                       splits > 1 ? part : y, N, K, M, row_offset, tiles_m, tiles_n, per, splits > 1 ? mn : 0ull);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_splitk_reduce(part, y, mn, splits, st);
}

using plan::TilePlan;

template <uint32_t WT, uint32_t XT>
hipError_t dispatch_x(const void* w, const void* x, float* y, uint32_t N, uint32_t K, uint32_t M,
                      uint32_t row_offset, const TilePlan& t, float* part, hipStream_t st) {
    if (WT == kGgmlQ8_0 && (K % kBK) != 0) {
        const uint64_t threads = (uint64_t)M * N;
        hipLaunchKernelGGL((gemm_q_generic<WT, XT>), dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0,
                           st, (const uint8_t*)w, x, y, N, K, M, row_offset);
        return hipGetLastError();
    }
    if (t.bm == 256) return launch_tiled<WT, XT, 256, 256>(w, x, y, N, K, M, row_offset, t.splits, part, st);
    if (t.bm == 128) return launch_tiled<WT, XT, 128, 128>(w, x, y, N, K, M, row_offset, t.splits, part, st);
    return launch_tiled<WT, XT, 64, 64>(w, x, y, N, K, M, row_offset, t.splits, part, st);
}

template <uint32_t WT>
hipError_t dispatch_w(const void* w, uint32_t xtype, const void* x, float* y, uint32_t N, uint32_t K,
                      uint32_t M, uint32_t row_offset, const TilePlan& t, float* part, hipStream_t st) {
    switch (xtype) {
        case kGgmlF32: return dispatch_x<WT, kGgmlF32>(w, x, y, N, K, M, row_offset, t, part, st);
        case kGgmlF16: return dispatch_x<WT, kGgmlF16>(w, x, y, N, K, M, row_offset, t, part, st);
        default: return dispatch_x<WT, kGgmlBF16>(w, x, y, N, K, M, row_offset, t, part, st);
    }
}

// f32 -> bf16 with round to nearest even (NaN stays NaN), 4 values per thread
__global__ void __launch_bounds__(256) f32_to_bf16_kernel(const float* __restrict__ x, uint32_t* __restrict__ y,
                                                          size_t n4) {
    const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n4) return;
    const u32x4 v = *(const u32x4*)(x + 4 * i);
    auto rn = [](uint32_t b) -> uint32_t {
        if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;  // quiet NaN
        return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
    };
    *(u32x2*)(y + 2 * i) = u32x2{rn(v.x) | (rn(v.y) << 16), rn(v.z) | (rn(v.w) << 16)};
}

// f32 -> fp16 with round to nearest even, the reference's float16_t(x) of
// the GEMM activations (llm.slang:1673); 8 values per thread
__global__ void __launch_bounds__(256) f32_to_f16_kernel(const float* __restrict__ x, u32x4* __restrict__ y,
                                                         size_t n8) {
    const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n8) return;
    const f32x4 a = *(const f32x4*)(x + 8 * i), b = *(const f32x4*)(x + 8 * i + 4);
    y[i] = u32x4{pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y), pack_f16x2(b.z, b.w)};
}

hipError_t convert_activations(const void* x, uint32_t xtype, void* out, uint32_t otype, size_t n, hipStream_t st) {
    (void)xtype;  // f32
    if (otype == kGgmlBF16) {
        const size_t n4 = n / 4;
        hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((uint32_t)((n4 + 255) / 256)), dim3(256), 0, st,
                           (const float*)x, (uint32_t*)out, n4);
    } else {
        const size_t n8 = n / 8;
        hipLaunchKernelGGL(f32_to_f16_kernel, dim3((uint32_t)((n8 + 255) / 256)), dim3(256), 0, st,
                           (const float*)x, (u32x4*)out, n8);
    }
    return hipGetLastError();
}

// y = silu(g) * u elementwise (the SwiGLU of two separately computed GEMMs)
__global__ void __launch_bounds__(256) swiglu_combine_kernel(const float* __restrict__ g,
                                                             const float* __restrict__ u, float* __restrict__ y,
                                                             size_t n) {
    const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) y[i] = silu(g[i]) * u[i];
}

using plan::align256;
using plan::GemmPlan;
using plan::kW16MinTokens;
using plan::plan_gemm;
using plan::row_bytes_of;

// Whether the fused SwiGLU kernel takes this launch: four features per
// lane store (N % 4 == 0) and 32-bit buffer offsets for the 16-bit
// activations and each weight.
bool swiglu_fused(uint32_t wtype, uint32_t N, uint32_t K, uint32_t M) {
    const uint64_t rb = row_bytes_of(wtype, K);
    return N % 4 == 0 && (K % kBK) == 0 && (uint64_t)M * K * 2u < (1ull << 31) && (uint64_t)N * rb < (1ull << 31);
}

}  // namespace

size_t batch_matmul_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, uint32_t M,
                                    int num_cus, size_t ws_limit) {
    if (M == 0 || N == 0 || (wtype == kGgmlQ4K && M <= kGemvMaxTokens)) return 0;
    return plan_gemm(wtype, xtype, N, K, M, num_cus, ws_limit).ws;
}

namespace {

// The LoRA GEMM's plan: the two-pass GEMM whose image carries the adapter.
GemmPlan lora_plan(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, uint32_t M, uint32_t rank, int num_cus) {
    GemmPlan p{};
    if (rank == 0 || rank > kLoraImageMaxRank || M == 0 || N == 0) return p;
    if (wtype == kGgmlQ4K && M <= kGemvMaxTokens) return p;
    p = plan_gemm(wtype, xtype, N, K, M, num_cus, kNoWorkspaceLimit);
    if (!p.two_pass) p = GemmPlan{};
    return p;
}

}  // namespace

size_t batch_matmul_lora_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, uint32_t M,
                                         uint32_t rank, int num_cus) {
    return lora_plan(wtype, xtype, N, K, M, rank, num_cus).ws;
}

hipError_t launch_batch_matmul_lora(const void* w, uint32_t wtype, const void* x, uint32_t xtype, float* y,
                                    uint32_t N, uint32_t K, uint32_t M, uint32_t row_offset, const LoraGemm& l,
                                    int num_cus, void* ws, hipStream_t st) {
    const GemmPlan pl = lora_plan(wtype, xtype, N, K, M, l.rank, num_cus);
    if (!pl.two_pass) return hipErrorNotSupported;
    const void* x16 = x;
    hipError_t e = hipSuccess;
    if (pl.convert_x) {
        x16 = (uint8_t*)ws + pl.x16_off;
        if ((e = convert_activations(x, xtype, (void*)x16, pl.xt, (size_t)M * K, st)) != hipSuccess) return e;
    }
    void* img = (uint8_t*)ws + pl.img_off;
    if ((e = launch_w16_image_lora(w, wtype, pl.xt, img, N, K, row_offset, l, st)) != hipSuccess) return e;
    const uint32_t tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
    PersistArgs a{};
    a.p[0] = PersistProblem{(const uint8_t*)img, x16, y, nullptr, nullptr, M, 0u, tiles_m};
    a.N = N;
    a.K = K;
    a.tiles_m = tiles_m;
    a.tiles_n = tiles_n;
    a.epi = kEpiStore;
    a.ldy = N;
    return launch_w16_gemm(a, pl.xt, false, false, num_cus, st);
}

size_t swiglu_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t out_dim, uint32_t in_dim,
                              uint32_t seq_len, int num_cus) {
    const uint32_t N = out_dim, K = in_dim, M = seq_len;
    if (!swiglu_fused(wtype, N, K, M)) {
        const size_t gu = 2 * align256((size_t)M * N * sizeof(float));
        return gu + batch_matmul_workspace_bytes(wtype, xtype, N, K, M, num_cus);
    }
    const size_t x16 = xtype == kGgmlF32 ? align256((size_t)M * K * 2u) : 0u;
    return x16 + (M >= kW16MinTokens ? w16_image_bytes(N, K, true) : 0u);
}

hipError_t launch_batch_matmul_swiglu(const void* wg, const void* wu, uint32_t wtype, const void* x,
                                      uint32_t xtype, float* y, uint32_t out_dim, uint32_t in_dim,
                                      uint32_t seq_len, int num_cus, void* ws, hipStream_t st) {
    if (seq_len == 0 || out_dim == 0) return hipSuccess;
    const uint32_t N = out_dim, K = in_dim, M = seq_len;
    if (wtype != kGgmlQ8_0) return hipErrorInvalidValue;
    if (!swiglu_fused(wtype, N, K, M)) {
        // two GEMMs into the workspace, then the elementwise SwiGLU
        float* g = (float*)ws;
        float* u = (float*)((uint8_t*)ws + align256((size_t)M * N * sizeof(float)));
        void* gemm_ws = (uint8_t*)ws + 2 * align256((size_t)M * N * sizeof(float));
        hipError_t e = launch_batch_matmul(wg, wtype, x, xtype, g, N, K, M, 0, num_cus, gemm_ws, st);
        if (e == hipSuccess) e = launch_batch_matmul(wu, wtype, x, xtype, u, N, K, M, 0, num_cus, gemm_ws, st);
        if (e != hipSuccess) return e;
        const size_t n = (size_t)M * N;
        hipLaunchKernelGGL(swiglu_combine_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, st, g, u, y, n);
        return hipGetLastError();
    }
    const void* x16 = x;
    uint32_t xt = xtype;
    size_t off = 0;
    if (xtype == kGgmlF32) {  // activations rounded to bf16 once (range of f32 kept)
        hipError_t e = convert_activations(x, xtype, ws, kGgmlBF16, (size_t)M * K, st);
        if (e != hipSuccess) return e;
        x16 = ws;
        xt = kGgmlBF16;
        off = align256((size_t)M * K * 2u);
    }
    const uint32_t tiles_m = (M + 255) / 256, tiles_n = (N + 127) / 128;
    const uint32_t grid = (uint32_t)min((uint64_t)tiles_m * tiles_n, (uint64_t)num_cus);
    PersistArgs a{};
    a.p[0] = PersistProblem{(const uint8_t*)wg, x16, y, nullptr, nullptr, M, 0u, tiles_m};
    a.W2 = (const uint8_t*)wu;
    a.N = N;
    a.K = K;
    a.tiles_m = tiles_m;
    a.tiles_n = tiles_n;
    a.epi = kEpiStore;
    a.ldy = N;
    if (M >= kW16MinTokens) {
        void* img = (uint8_t*)ws + off;
        hipError_t e = launch_w16_image(wg, wu, wtype, xt, img, N, K, 0u, st);
        if (e != hipSuccess) return e;
        a.p[0].W = (const uint8_t*)img;
        a.W2 = nullptr;
        return launch_w16_gemm(a, xt, true, false, num_cus, st);
    }
    if (xt == kGgmlF16)
        hipLaunchKernelGGL((gemm_q_persist<kGgmlQ8_0, kGgmlF16, true>), dim3(grid), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_q_persist<kGgmlQ8_0, kGgmlBF16, true>), dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_batch_matmul(const void* w, uint32_t wtype, const void* x, uint32_t xtype,
                               float* y, uint32_t out_dim, uint32_t in_dim, uint32_t seq_len,
                               uint32_t row_offset, int num_cus, void* ws, hipStream_t st, size_t ws_limit) {
    if (seq_len == 0 || out_dim == 0) return hipSuccess;
    const uint32_t N = out_dim, K = in_dim, M = seq_len;
    if (wtype == kGgmlQ4K && M <= kGemvMaxTokens)
        return launch_gemv_q4k(w, xtype, x, y, N, K, M, row_offset, st);
    const GemmPlan pl = plan_gemm(wtype, xtype, N, K, M, num_cus, ws_limit);
    if (pl.few) return launch_gemm_few(w, wtype, x, xtype, y, N, K, M, row_offset, st);
    if (pl.skinny) return launch_gemm_skinny(w, wtype, x, xtype, y, N, K, M, row_offset, pl.splits, ws, st);
    if (!pl.persistent) {
        if (wtype == kGgmlQ8_0)
            return dispatch_w<kGgmlQ8_0>(w, xtype, x, y, N, K, M, row_offset, pl.tiles, (float*)ws, st);
        return dispatch_w<kGgmlQ4K>(w, xtype, x, y, N, K, M, row_offset, pl.tiles, (float*)ws, st);
    }
    const void* x16 = x;
    if (pl.convert_x) {
        x16 = (uint8_t*)ws + pl.x16_off;
        hipError_t e = convert_activations(x, xtype, (void*)x16, pl.xt, (size_t)M * K, st);
        if (e != hipSuccess) return e;
    }
    const uint32_t tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
    const uint32_t grid = (uint32_t)min((uint64_t)tiles_m * tiles_n, (uint64_t)num_cus);
    PersistArgs a{};
    a.p[0] = PersistProblem{(const uint8_t*)w, x16, y, nullptr, nullptr, M, row_offset, tiles_m};
    a.N = N;
    a.K = K;
    a.tiles_m = tiles_m;
    a.tiles_n = tiles_n;
    a.epi = kEpiStore;
    a.ldy = N;
    if (pl.two_pass) {
        void* img = (uint8_t*)ws + pl.img_off;
        hipError_t e = launch_w16_image(w, nullptr, wtype, pl.xt, img, N, K, row_offset, st);
        if (e != hipSuccess) return e;
        a.p[0].W = (const uint8_t*)img;
        return launch_w16_gemm(a, pl.xt, false, false, num_cus, st);
    }
    // Q8_0 on the 8-wave kernel (its half-row dequantization is lighter than
    // Q4_K's and it measures faster); Q4_K on the 4-wave one
    if (wtype == kGgmlQ8_0) {
        if (pl.xt == kGgmlF16)
            hipLaunchKernelGGL((gemm_q_persist8<kGgmlQ8_0, kGgmlF16>), dim3(grid), dim3(512), 0, st, a);
        else
            hipLaunchKernelGGL((gemm_q_persist8<kGgmlQ8_0, kGgmlBF16>), dim3(grid), dim3(512), 0, st, a);
    } else {
        if (pl.xt == kGgmlF16)
            hipLaunchKernelGGL((gemm_q_persist<kGgmlQ4K, kGgmlF16, false>), dim3(grid), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((gemm_q_persist<kGgmlQ4K, kGgmlBF16, false>), dim3(grid), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

namespace {

// Whether jobs [j0, j0 + n) (n <= 2) run as one persistent launch: 16-bit
// activations, N % 4 == 0, whole 64-wide K stages, 32-bit buffer offsets for
// every job's activations and used weight rows, and at least half the CUs'
// worth of 256 x 256 tiles between them.
bool multi_persistent(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, const GemmJob* jobs, uint32_t n,
                      int num_cus) {
    if (xtype == kGgmlF32 || N % 4 || K % kBK) return false;
    const uint64_t rb = row_bytes_of(wtype, K);
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < n; i++) {
        if ((uint64_t)jobs[i].M * K * 2u >= (1ull << 31) || (uint64_t)N * rb >= (1ull << 31)) return false;
        tiles += (uint64_t)((jobs[i].M + 255) / 256) * ((N + 255) / 256);
    }
    return 2 * tiles >= (uint64_t)num_cus;
}

// Whether a persistent job group runs two-pass (weight images): as a single
// GEMM, by its total tokens.
bool multi_two_pass(const GemmJob* jobs, uint32_t n) {
    uint64_t m = 0;
    for (uint32_t i = 0; i < n; i++) m += jobs[i].M;
    return m >= kW16MinTokens;
}

// Split-SwiGLU jobs (kEpiSplitSwiglu): N = split + 2 f weight rows, f gate
// rows after the plain ones, then f up rows. Their two-pass image is the
// plain image of the first split rows followed by the SwiGLU-arranged image
// of the gate and up rows (128 outputs per 256-row panel).
uint32_t swiglu_outputs(const GemmEpilogue& epi, uint32_t N) { return (N - epi.split) / 2u; }
size_t multi_image_bytes(const GemmEpilogue& epi, uint32_t N, uint32_t K) {
    if (epi.kind == kEpiSplitSwiglu)
        return w16_image_bytes(epi.split, K, false) + w16_image_bytes(swiglu_outputs(epi, N), K, true);
    return w16_image_bytes(N, K, false);
}
hipError_t build_split_swiglu_image(const GemmJob& j, uint32_t wtype, uint32_t otype, void* img, uint32_t N,
                                    uint32_t K, uint32_t split, hipStream_t st) {
    const uint64_t rb = row_bytes_of(wtype, K);
    const uint8_t* const w = (const uint8_t*)j.w + (uint64_t)j.row_offset * rb;
    const uint32_t f = (N - split) / 2u;
    if (split > 0)
        if (hipError_t e = launch_w16_image(w, nullptr, wtype, otype, img, split, K, 0u, st); e != hipSuccess)
            return e;
    return launch_w16_image(w + (uint64_t)split * rb, w + (uint64_t)(split + f) * rb, wtype, otype,
                            (uint8_t*)img + w16_image_bytes(split, K, false), f, K, 0u, st);
}

// Whether jobs [j0, j0 + n) run fused in one launch: the persistent
// kernels take them (split-SwiGLU: the two-pass one only, the one-pass
// kernels have no such epilogue).
bool multi_fused(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, const GemmJob* jobs, uint32_t n,
                 const GemmEpilogue& epi, int num_cus) {
    if (!multi_persistent(wtype, xtype, N, K, jobs, n, num_cus)) return false;
    // head routing: the two-pass kernel's epilogue
    if (epi.heads && !multi_two_pass(jobs, n)) return false;
    return epi.kind != kEpiSplitSwiglu || multi_two_pass(jobs, n);
}

PersistArgs multi_args(uint32_t N, uint32_t K, const GemmJob* jobs, uint32_t n, const GemmEpilogue& epi) {
    PersistArgs a{};
    const uint32_t tiles_n = (N + 255) / 256;
    uint32_t tiles_m = 0;
    for (uint32_t i = 0; i < n; i++) {
        const GemmJob& j = jobs[i];
        const uint32_t tm = (j.M + 255) / 256;
        a.p[i] = PersistProblem{(const uint8_t*)j.w, j.x, j.y, j.gate, j.y2, j.M, j.row_offset, tm};
        tiles_m += tm;
    }
    a.N = N;
    a.K = K;
    a.tiles_m = tiles_m;
    a.tiles_n = tiles_n;
    a.epi = epi.kind;
    a.ldy = epi.ldy;
    a.ldy2 = epi.ldy2;
    a.split = epi.kind == kEpiSplitGelu || epi.kind == kEpiSplitSwiglu ? epi.split : N;
    a.y2_bf16 = epi.y2_type == kGgmlBF16 ? 1u : 0u;
    if (const GemmHeads* h = epi.heads) {
        a.heads = HeadsEpi{h->q, h->k, h->v, h->cos, h->sin, {}, {}, {}, h->n_heads, h->seq,
                           h->otype == kGgmlBF16 ? 1u : 0u, h->eps};
        for (uint32_t i = 0; i < n; i++) {
            a.heads.qn[i] = jobs[i].q_norm;
            a.heads.kn[i] = jobs[i].k_norm;
            a.heads.row0[i] = jobs[i].row0;
        }
    }
    if (epi.kind == kEpiSplitSwiglu)  // the plain panels, then the SwiGLU ones
        a.tiles_n = epi.split / 256u + (swiglu_outputs(epi, N) + 127u) / 128u;
    return a;
}

template <uint32_t WT, uint32_t XT>
hipError_t launch_persist_multi(const PersistArgs& a, int num_cus, hipStream_t st) {
    const uint32_t grid = (uint32_t)min((uint64_t)a.tiles_m * a.tiles_n, (uint64_t)num_cus);
    if constexpr (WT == kGgmlQ8_0) {
        auto kern = a.epi == kEpiResidual    ? gemm_q_persist8<WT, XT, kEpiResidual, true>
                    : a.epi == kEpiSplitGelu ? gemm_q_persist8<WT, XT, kEpiSplitGelu, true>
                                             : gemm_q_persist8<WT, XT, kEpiStore, true>;
        hipLaunchKernelGGL(kern, dim3(grid), dim3(512), 0, st, a);
    } else {
        auto kern = a.epi == kEpiResidual    ? gemm_q_persist<WT, XT, false, kEpiResidual, true>
                    : a.epi == kEpiSplitGelu ? gemm_q_persist<WT, XT, false, kEpiSplitGelu, true>
                                             : gemm_q_persist<WT, XT, false, kEpiStore, true>;
        hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

// One job the persistent kernel does not take: the plain GEMM into the
// workspace `t` (directly into the output for an unstrided store), then
// the epilogue as glue passes. `gemm_ws` is the GEMM's own workspace.
hipError_t run_job_fallback(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, const GemmJob& j,
                            const GemmEpilogue& epi, int num_cus, float* t, void* gemm_ws, hipStream_t st) {
    if (epi.kind == kEpiStore && epi.ldy == N)
        return launch_batch_matmul(j.w, wtype, j.x, xtype, j.y, N, K, j.M, j.row_offset, num_cus, gemm_ws, st);
    hipError_t e = launch_batch_matmul(j.w, wtype, j.x, xtype, t, N, K, j.M, j.row_offset, num_cus, gemm_ws, st);
    if (e != hipSuccess) return e;
    if (epi.kind == kEpiResidual) {
        ResidualArgs r{j.y, t, nullptr, j.gate, epi.ldy, N, j.M, N, 0.0f};
        r.grid_cus = (uint32_t)num_cus;
        return launch_residual(r, false, st);
    }
    if (const GemmHeads* h = epi.heads) {  // columns [0, split) into the heads
        const QkvHeadsArgs q{t, j.q_norm, j.k_norm, h->cos, h->sin, h->q, h->k, h->v, N, j.M, h->n_heads, h->seq,
                             j.row0, h->eps};
        if ((e = launch_qkv_heads(q, h->otype, st)) != hipSuccess) return e;
    }
    if (epi.kind == kEpiSplitSwiglu) {  // columns [0, split) copied, then silu(gate) * up
        const uint32_t f = swiglu_outputs(epi, N);
        if (epi.split > 0 && !epi.heads) {
            const ActColsArgs c{t, j.y, N, 0u, 0u, epi.ldy, 0u, j.M, epi.split};
            if ((e = launch_act_cols(c, kActCopy, kGgmlF32, st)) != hipSuccess) return e;
        }
        const ActColsArgs c{t, j.y2, N, epi.split, epi.split + f, epi.ldy2, 0u, j.M, f};
        return launch_act_cols(c, kActSiluMul, epi.y2_type, st);
    }
    const uint32_t split = epi.kind == kEpiSplitGelu ? epi.split : N;
    if (split > 0 && !epi.heads) {
        const ActColsArgs c{t, j.y, N, 0u, 0u, epi.ldy, 0u, j.M, split};
        if ((e = launch_act_cols(c, kActCopy, kGgmlF32, st)) != hipSuccess) return e;
    }
    if (split < N) {
        const ActColsArgs c{t, j.y2, N, split, 0u, epi.ldy2, 0u, j.M, N - split};
        e = launch_act_cols(c, kActGelu, epi.y2_type, st);
    }
    return e;
}

// Workspace of the fallback jobs: the largest job's f32 result (when the
// epilogue is not a plain store), then the largest GEMM workspace.
size_t fallback_t_bytes(uint32_t N, const GemmJob* jobs, uint32_t n_jobs, const GemmEpilogue& epi,
                        uint32_t wtype, uint32_t xtype, uint32_t K, int num_cus) {
    size_t t = 0;
    for (uint32_t i = 0; i < n_jobs; i += 2) {
        const uint32_t n = min(2u, n_jobs - i);
        if (multi_fused(wtype, xtype, N, K, jobs + i, n, epi, num_cus)) continue;
        if (epi.kind == kEpiStore && epi.ldy == N) continue;
        for (uint32_t q = i; q < i + n; q++) t = max(t, align256((size_t)jobs[q].M * N * sizeof(float)));
    }
    return t;
}

}  // namespace

size_t batch_matmul_multi_workspace_bytes(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K,
                                          const GemmJob* jobs, uint32_t n_jobs, const GemmEpilogue& epi,
                                          int num_cus, bool prebuilt_images) {
    const size_t t = fallback_t_bytes(N, jobs, n_jobs, epi, wtype, xtype, K, num_cus);
    size_t need = 0;
    for (uint32_t i = 0; i < n_jobs; i += 2) {
        const uint32_t n = min(2u, n_jobs - i);
        if (multi_fused(wtype, xtype, N, K, jobs + i, n, epi, num_cus)) {
            if (multi_two_pass(jobs + i, n) && !prebuilt_images) need = max(need, n * multi_image_bytes(epi, N, K));
            continue;
        }
        for (uint32_t q = i; q < i + n; q++)
            need = max(need, t + batch_matmul_workspace_bytes(wtype, xtype, N, K, jobs[q].M, num_cus));
    }
    return need;
}

// Next-group image items one idle workgroup of a two-pass GEMM takes on:
// one per four of the GEMM's K stages for Q4_K items (an item is 4 stages
// of a 256-row panel, read as packed weights and written as 16-bit
// operands: ~6 us on a CU beside the GEMM, a tile stage ~1.5 us), one per
// eight for Q8_0 items (68 bytes a row and stage against 36), so the items
// end within the idle workgroups' last-round time.
uint32_t next_items_per_idle_wg(uint32_t K, uint32_t wtype) {
    return max(1u, K / (uint32_t)kBK / (wtype == kGgmlQ8_0 ? 8u : 4u));
}

uint32_t next_image_items(const NextImageSet& nx) {
    uint32_t all = 0;
    for (uint32_t i = 0; i < nx.count; i++) all += w16_image_items(nx.N[i], nx.K[i], nx.sw[i] != 0);
    return all;
}

// The raw rows of next image i: plain, w at its row_offset (g, u null
// pointers returned as g = w); SwiGLU, its gate rows g and up rows u.
static void next_image_rows(const NextImageSet& nx, uint32_t i, const void*& g, const void*& u) {
    if (!nx.sw[i]) {
        g = nx.w[i];
        u = nullptr;
        return;
    }
    const uint64_t rb = row_bytes_of(nx.wtype, nx.K[i]);
    g = (const uint8_t*)nx.w[i] + (uint64_t)nx.row_offset[i] * rb;
    u = (const uint8_t*)g + (uint64_t)(nx.up[i] ? nx.up[i] : nx.N[i]) * rb;
}

// Later groups' images: the items [0, fused) came from the GEMM's idle
// workgroups; the rest of each image here.
hipError_t finish_next_images(const NextImageSet& nx, uint32_t otype, uint32_t fused, hipStream_t st) {
    uint32_t first = 0;
    for (uint32_t i = 0; i < nx.count; i++) {
        const uint32_t per = w16_image_items(nx.N[i], nx.K[i], nx.sw[i] != 0);
        const uint32_t done = fused > first ? min(per, fused - first) : 0u;
        first += per;
        if (done == per) continue;
        const void *g, *u;
        next_image_rows(nx, i, g, u);
        const hipError_t e = launch_w16_image(g, u, nx.wtype, otype, nx.img[i], nx.N[i], nx.K[i],
                                              nx.sw[i] ? 0u : nx.row_offset[i], st, done);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_batch_matmul_multi(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, const GemmJob* jobs,
                                     uint32_t n_jobs, const GemmEpilogue& epi, int num_cus, void* ws,
                                     hipStream_t st, const void* const* images, const NextImageSet* next) {
    if (next && (next->count == 0 || next->count > kMaxNextImages || (xtype != kGgmlF16 && xtype != kGgmlBF16)))
        return hipErrorInvalidValue;
    uint32_t fused = 0;  // next-image items the last group's GEMM builds
    // a group of Q4_K projections of a few tokens (the per-block
    // modulation vectors) as one GEMV launch
    if (wtype == kGgmlQ4K && epi.kind == kEpiStore && n_jobs > 1) {
        const hipError_t e = launch_gemv_q4k_multi(xtype, jobs, n_jobs, N, K, epi.ldy, st);
        if (e != hipErrorNotSupported) return e != hipSuccess || !next ? e : finish_next_images(*next, xtype, 0, st);
    }
    const size_t t_bytes = fallback_t_bytes(N, jobs, n_jobs, epi, wtype, xtype, K, num_cus);
    for (uint32_t i = 0; i < n_jobs; i += 2) {
        const uint32_t n = min(2u, n_jobs - i);
        hipError_t e = hipSuccess;
        if (multi_fused(wtype, xtype, N, K, jobs + i, n, epi, num_cus)) {
            PersistArgs a = multi_args(N, K, jobs + i, n, epi);
            if (multi_two_pass(jobs + i, n)) {
                const size_t img_bytes = multi_image_bytes(epi, N, K);
                for (uint32_t q = 0; q < n && e == hipSuccess; q++) {
                    if (images) {  // built ahead by the caller (launch_w16_image, same arguments)
                        a.p[q].W = (const uint8_t*)images[i + q];
                        continue;
                    }
                    void* img = (uint8_t*)ws + q * img_bytes;
                    e = epi.kind == kEpiSplitSwiglu
                            ? build_split_swiglu_image(jobs[i + q], wtype, xtype, img, N, K, epi.split, st)
                            : launch_w16_image(jobs[i + q].w, nullptr, wtype, xtype, img, N, K,
                                               jobs[i + q].row_offset, st);
                    a.p[q].W = (const uint8_t*)img;
                }
                const uint64_t tiles = (uint64_t)a.tiles_m * a.tiles_n;
                if (next && i + n == n_jobs && tiles % (uint64_t)num_cus != 0) {
                    const uint32_t idle = num_cus - (uint32_t)(tiles % (uint64_t)num_cus);
                    fused = min(next_image_items(*next), idle * next_items_per_idle_wg(K, next->wtype));
                    NextImages& ni = a.next;
                    uint32_t first = 0;
                    for (uint32_t q = 0; q < next->count; q++) {
                        const void *g, *u;
                        next_image_rows(*next, q, g, u);
                        ni.W[q] = (const uint8_t*)g;
                        ni.W2[q] = (const uint8_t*)u;
                        ni.img[q] = (uint8_t*)next->img[q];
                        ni.row_offset[q] = next->sw[q] ? 0u : next->row_offset[q];
                        ni.N[q] = next->N[q];
                        ni.K[q] = next->K[q];
                        ni.first[q] = first;
                        first += w16_image_items(next->N[q], next->K[q], next->sw[q] != 0);
                    }
                    ni.count = next->count;
                    ni.wtype = next->wtype;
                    ni.items = fused;
                }
                if (e == hipSuccess) e = launch_w16_gemm(a, xtype, false, n == 2, num_cus, st);
            } else if (wtype == kGgmlQ8_0) {
                e = xtype == kGgmlF16 ? launch_persist_multi<kGgmlQ8_0, kGgmlF16>(a, num_cus, st)
                                      : launch_persist_multi<kGgmlQ8_0, kGgmlBF16>(a, num_cus, st);
            } else {
                e = xtype == kGgmlF16 ? launch_persist_multi<kGgmlQ4K, kGgmlF16>(a, num_cus, st)
                                      : launch_persist_multi<kGgmlQ4K, kGgmlBF16>(a, num_cus, st);
            }
        } else {
            for (uint32_t q = i; q < i + n && e == hipSuccess; q++)
                e = run_job_fallback(wtype, xtype, N, K, jobs[q], epi, num_cus, (float*)ws,
                                     (uint8_t*)ws + t_bytes, st);
        }
        if (e != hipSuccess) return e;
    }
    return next ? finish_next_images(*next, xtype, fused, st) : hipSuccess;
}

}  // namespace llmr
