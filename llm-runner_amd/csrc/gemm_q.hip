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

// 16-byte chunk c (0..7) of LDS row r (128-byte rows).
__device__ __forceinline__ uint32_t lds_off(uint32_t r, uint32_t c) {
    return r * 128u + ((c ^ (r & 7u)) << 4);
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
            lo[2 * i] = pack_f16x2(dsc0 * (float)(l4 & 0xffu) - dmn0,
                                   dsc0 * (float)((l4 >> 8) & 0xffu) - dmn0);
            lo[2 * i + 1] = pack_f16x2(dsc0 * (float)((l4 >> 16) & 0xffu) - dmn0,
                                       dsc0 * (float)(l4 >> 24) - dmn0);
            hi[2 * i] = pack_f16x2(dsc1 * (float)(h4 & 0xffu) - dmn1,
                                   dsc1 * (float)((h4 >> 8) & 0xffu) - dmn1);
            hi[2 * i + 1] = pack_f16x2(dsc1 * (float)((h4 >> 16) & 0xffu) - dmn1,
                                       dsc1 * (float)(h4 >> 24) - dmn1);
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
    if (wgs(256, 256) >= want) return launch_tiled<WT, XT, 256, 256>(w, x, y, N, K, M, row_offset, st);
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
