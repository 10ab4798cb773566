// gemm_few.hip - dequant-GEMM for few tokens (M <= 256) with enough output
// features to give at least every other CU a 32 x 96 tile: batch_matmul_q8 /
// batch_matmul_q4k (llm.slang:1639-1767, :2277-2365), e.g. the single Q8_0
// linear of 256 tokens x 3072 -> 3072 with f32 activations.
//
//   Y[m, n] = sum_k X[m, k] * W[row_offset + n, k]     (f32 out, row stride N)
//
// One launch, no workspace. What bounds such a launch is the bytes every CU
// pulls from L2 (~90 GB/s per CU with one workgroup per CU, ~23 TB/s over
// the device, by a read-bandwidth probe on MI355X), not the matrix cores. A
// CU that owns T tokens x F features over the whole K reads K (T xb + F wb)
// bytes (xb = 4 for f32 activations, wb = 34/32 for Q8_0) with T F = M N /
// CUs; 32 x 96 is the smallest such read for 256 x 3072 on 256 CUs (706 KiB
// per CU at K = 3072). Splitting K across CUs would cut that by sqrt(splits)
// but adds the partial sums' round trip through memory and a second launch.
//
// Workgroup = 8 waves (two per SIMD) over one 32-token x 96-feature tile;
// wave w takes the K stages w, w + 8, w + 16, ... (64 k each) and keeps the
// whole tile in three 32x32x16 MFMA accumulators; at the end the eight
// partial tiles meet in LDS and are summed in wave order (deterministic).
// (Twelve waves, with half again as many loads in flight per CU, measured
// slower: the load path's throughput is the bound, not its latency.)
//  * Loads are laid out for the memory system, not for the MFMA: a load
//    instruction of a wave reads 4 activation rows x 256 bytes (f32; 8 rows
//    x 128 bytes for 16-bit) or 12 weight rows x 80 bytes (Q8_0: the
//    stage's 68 and 12 of the next; Q4_K: 16 rows x 48 bytes). Loaded with the
//    MFMA's lane layout (lane = row: 32 rows x 32 bytes per instruction)
//    the same bytes came at a third of the rate (32 against 74-86 GB/s per
//    CU, read-pattern probe on MI355X): a CU's vector memory path handles
//    about one cache line per clock, whatever part of it is used.
//  * Each wave stages its stage in its own LDS region (no workgroup barrier
//    in the loop; a wave's LDS accesses run in order): activations rounded
//    to the operand type on the way in (fp16 against Q8_0, the reference's
//    float16_t(x); bf16 against Q4_K, whose reference keeps x in f32) as 32
//    rows x 128 bytes with the GEMM kernels' chunk swizzle; the packed
//    weight bytes as they are (Q8_0: 80 bytes per row, 68 of them used;
//    Q4_K: the 16-byte header and the quarter's 32 quant bytes at 64).
//  * The next stage's loads are in flight while this stage is read back in
//    MFMA layout (lane (r = lane % 32, h = lane / 32): token / feature row r,
//    k [32 h, 32 h + 32) of the stage) and multiplied; the weights are
//    dequantized per k step in registers with the other kernels' operand
//    code (q8x8_f16 / fma_pair: the same operand bits). k step t multiplies
//    k_local = 32 h + 8 t + i (i = 0..7) for both operands.
// Rows past M or N read as zero through range-limited buffer descriptors and
// are not stored.
// Tile order: when the tile count is a multiple of 8, the 8 XCDs (workgroup
// b runs on XCD b % 8) each take a contiguous eighth of the feature-major
// tile list, so an XCD's L2 holds a slice of the weight and all the
// activations instead of the whole weight.
#include "gemm_q_common.h"
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

constexpr uint32_t kFT = plan::kFewTokens, kFF = plan::kFewFeatures, kFB = kFF / 32u;  // 3 feature blocks
constexpr uint32_t kFewWaves = 8;  // two per SIMD
constexpr uint32_t kRedLd = kFF + 4u;  // floats per LDS row of a partial tile (16-byte pad)
static_assert(kFT == 32 && kFF % 32 == 0, "one 32-token block, whole 32-feature blocks");

// A lane's packed weight bytes of one stage and feature block, as read back
// from the wave's LDS region.
template <uint32_t WT>
struct FewW;
// Q8_0 block 2 s + h: 9 dwords from the block's dword-aligned start (byte 0
// of the row's 68 for h = 0, byte 32 for h = 1, where the block starts 2
// bytes in).
template <>
struct FewW<kGgmlQ8_0> {
    static constexpr uint32_t kRow = 80;  // LDS bytes per weight row (68 used)
    u32x4 a, b;
    uint32_t e;
    __device__ __forceinline__ void read(const uint8_t* ws, uint32_t row, uint32_t h) {
        const uint8_t* p = ws + row * kRow + 32u * h;
        a = *(const u32x4*)p;
        b = *(const u32x4*)(p + 16);
        e = *(const uint32_t*)(p + 32);
    }
    __device__ __forceinline__ uint32_t word(uint32_t i) const { return i < 4 ? a[i] : i < 8 ? b[i - 4] : e; }
};
// Q4_K: the superblock's 16-byte header and quarter s % 4's 32 quant bytes.
template <>
struct FewW<kGgmlQ4K> {
    static constexpr uint32_t kRow = 64;  // header, 32 quant bytes, 16 unused
    u32x4 hdr, qa, qb;
    __device__ __forceinline__ void read(const uint8_t* ws, uint32_t row, uint32_t) {
        const uint8_t* p = ws + row * kRow;
        hdr = *(const u32x4*)p;
        qa = *(const u32x4*)(p + 16);
        qb = *(const u32x4*)(p + 32);
    }
};

// A wave's loads of one stage, in the memory-friendly layout: lane l of
// activation load i holds row 4 i + l / 16, bytes 16 (l % 16) of the stage
// (f32) or row 8 i + l / 8, bytes 16 (l % 8) (16-bit); lane l < 60 of Q8_0
// weight load j holds row 12 j + l / 5, bytes 16 p (p = l % 5 < 4) or 52..67
// (p = 4, of which the last dword is kept) of the row's 68 bytes of the
// stage (no read crosses them); lane l of Q4_K weight load j holds row
// 16 j + l / 4, piece l % 4 (0 the superblock header, 1-2 the quarter's
// quants, 3 nothing).
template <uint32_t WT, uint32_t XT>
struct FewLoads {
    static constexpr uint32_t kXi = XT == kGgmlF32 ? 8u : 4u, kWj = WT == kGgmlQ8_0 ? 8u : 6u;
    u32x4 x[kXi], w[kWj];
    __device__ __forceinline__ void load(rsrc_t xr, rsrc_t wr, uint32_t m_row, uint32_t K, uint64_t rb,
                                         uint32_t s, uint32_t lane) {
        if constexpr (XT == kGgmlF32) {
#pragma unroll
            for (uint32_t i = 0; i < kXi; i++)
                x[i] = bload16(xr, (m_row + 4u * i + (lane >> 4)) * K * 4u + 16u * (lane & 15u), 256u * s);
        } else {
#pragma unroll
            for (uint32_t i = 0; i < kXi; i++)
                x[i] = bload16(xr, (m_row + 8u * i + (lane >> 3)) * K * 2u + 16u * (lane & 7u), 128u * s);
        }
        if constexpr (WT == kGgmlQ8_0) {
            const uint32_t q = lane / 5u, p = lane - 5u * q;  // row within the load, piece
            const uint32_t po = p < 4u ? 16u * p : 52u;
#pragma unroll
            for (uint32_t j = 0; j < kWj; j++)
                w[j] = bload16(wr, lane < 60u ? (uint32_t)((12u * j + q) * rb) + po : 0x80000000u, 68u * s);
        } else {
            const uint32_t p = lane & 3u, sh = (s >> 2) * 144u;
            const uint32_t off = p == 0 ? sh : p < 3 ? sh + 16u + 32u * (s & 3u) + 16u * (p - 1u) : 0x80000000u;
#pragma unroll
            for (uint32_t j = 0; j < kWj; j++) {
                const uint32_t row = 16u * j + (lane >> 2);
                w[j] = bload16(wr, p < 3 ? (uint32_t)(row * rb) + off : off, 0u);
            }
        }
    }
    // into the wave's LDS region: activations rounded to OT (xs, 32 rows x
    // 128 bytes, swizzled chunks), weight bytes as they are (ws). Q8_0: every
    // lane writes a 16-byte piece and a dword, the ones it has nothing for
    // into the region's pad (no branch: a divergent one in this loop made
    // every wait on the loads a full drain)
    template <uint32_t OT>
    __device__ __forceinline__ void store(uint8_t* xs, uint8_t* ws, uint32_t lane) const {
        if constexpr (XT == kGgmlF32) {
#pragma unroll
            for (uint32_t i = 0; i < kXi; i++) {
                const uint32_t row = 4u * i + (lane >> 4), c16 = lane & 15u;
                const f32x4 v = __builtin_bit_cast(f32x4, x[i]);
                const u32x2 o = OT == kGgmlBF16 ? u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)}
                                                : u32x2{pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w)};
                *(u32x2*)(xs + lds_off(row, c16 >> 1) + 8u * (c16 & 1u)) = o;
            }
        } else {
#pragma unroll
            for (uint32_t i = 0; i < kXi; i++) *(u32x4*)(xs + lds_off(8u * i + (lane >> 3), lane & 7u)) = x[i];
        }
        constexpr uint32_t kRow = FewW<WT>::kRow;
        if constexpr (WT == kGgmlQ8_0) {
            const uint32_t q = lane / 5u, p = lane - 5u * q;
            const bool piece = lane < 60u && p < 4u, last = lane < 60u && p == 4u;
#pragma unroll
            for (uint32_t j = 0; j < kWj; j++) {
                const uint32_t row = (12u * j + q) * kRow;
                *(u32x4*)(ws + (piece ? row + 16u * p : kFF * kRow)) = w[j];
                *(uint32_t*)(ws + (last ? row + 64u : kFF * kRow)) = w[j].w;
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kWj; j++)
                *(u32x4*)(ws + (16u * j + (lane >> 2)) * kRow + 16u * (lane & 3u)) = w[j];
        }
    }
};

// The weight operands of one stage and feature block, per k step, built
// from the raw words when the step needs them (no realigned copy of the
// stage is kept: registers are the limit here).
template <uint32_t WT, uint32_t OT>
struct FewWop;
template <uint32_t OT>
struct FewWop<kGgmlQ8_0, OT> {
    float s, b;  // bf16: (2^24 d, -128 d); f16: (d, -)
    __device__ __forceinline__ void prepare(const FewW<kGgmlQ8_0>& w, uint32_t h, uint32_t) {
        // the block's scale: low half of dword 0 (h = 0) or high half (h = 1)
        const float d = f16_bits_to_f32((w.word(0) >> (16u * h)) & 0xffffu);
        if constexpr (OT == kGgmlBF16) {
            s = d * 16777216.0f;
            b = -128.0f * d;
        } else {
            s = d;
            b = 0.0f;
        }
    }
    // quants 8 t .. 8 t + 7 of the block: dwords 2 t, 2 t + 1 after the
    // realignment (byte 2 of the loaded words for h = 0, byte 4 for h = 1)
    __device__ __forceinline__ f16x8 op(const FewW<kGgmlQ8_0>& w, uint32_t t, uint32_t sel) const {
        const uint32_t q0 = __builtin_amdgcn_perm(w.word(2 * t + 1), w.word(2 * t), sel);
        const uint32_t q1 = __builtin_amdgcn_perm(w.word(2 * t + 2), w.word(2 * t + 1), sel);
        if constexpr (OT == kGgmlBF16) {
            // RN_bf16(d q): q + 128 read as a subnormal half, d q = (2^24 d) h - 128 d
            // exactly in f32, then one rounding (WRow<Q8_0>::chunk)
            const uint32_t u0 = q0 ^ 0x80808080u, u1 = q1 ^ 0x80808080u;
            return __builtin_bit_cast(f16x8, u32x4{fma_pair<OT>(sub16x2(u0, kSelLo), s, b),
                                                   fma_pair<OT>(sub16x2(u0, kSelHi), s, b),
                                                   fma_pair<OT>(sub16x2(u1, kSelLo), s, b),
                                                   fma_pair<OT>(sub16x2(u1, kSelHi), s, b)});
        } else {
            const _Float16 hs = (_Float16)s;
            return __builtin_bit_cast(f16x8, q8x8_f16(q0, q1, f16x2{hs, hs}));
        }
    }
};
template <uint32_t OT>
struct FewWop<kGgmlQ4K, OT> {
    float s, b;  // RN(s q' + b): q' = q 2^-24 (low nibble) or 16 q 2^-24 (high nibble)
    __device__ __forceinline__ void prepare(const FewW<kGgmlQ4K>& w, uint32_t h, uint32_t j) {
        const float d = f16_bits_to_f32(w.hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(w.hdr.x >> 16);
        uint32_t sc, mn;
        q4k_scale_min(2u * j + h, w.hdr.y, w.hdr.z, w.hdr.w, sc, mn);
        s = d * (float)sc * (h ? 1048576.0f : 16777216.0f);
        b = -(dmin * (float)mn);
    }
    // quant bytes 8 t .. 8 t + 7 of the quarter, nibble h masked in place
    __device__ __forceinline__ f16x8 op(const FewW<kGgmlQ4K>& w, uint32_t t, uint32_t mask) const {
        const uint32_t q0 = (t < 2 ? w.qa[2 * t] : w.qb[2 * t - 4]) & mask;
        const uint32_t q1 = (t < 2 ? w.qa[2 * t + 1] : w.qb[2 * t - 3]) & mask;
        return __builtin_bit_cast(f16x8, u32x4{fma_pair<OT>(sub16x2(q0, kSelLo), s, b),
                                               fma_pair<OT>(sub16x2(q0, kSelHi), s, b),
                                               fma_pair<OT>(sub16x2(q1, kSelLo), s, b),
                                               fma_pair<OT>(sub16x2(q1, kSelHi), s, b)});
    }
};

template <uint32_t WT, uint32_t XT>
__global__ void __launch_bounds__(kFewWaves * 64u, 1)
    gemm_q_few(const uint8_t* __restrict__ W, const void* __restrict__ X, float* __restrict__ Y, uint32_t N,
               uint32_t K, uint32_t M, uint32_t row_offset, uint32_t tiles_m, uint32_t tiles_n) {
    constexpr uint32_t OT = (XT == kGgmlBF16 || (XT == kGgmlF32 && WT == kGgmlQ4K)) ? kGgmlBF16 : kGgmlF16;
    // per wave: its stage's 16-bit activations (32 x 128 bytes) and packed
    // weight rows; after the loop, the waves' partial tiles
    constexpr uint32_t kXs = kFT * 128u, kWs = kFF * FewW<WT>::kRow + 16u, kWave = kXs + kWs;  // + a pad dword
    constexpr uint32_t kRed = kFewWaves * kFT * kRedLd * 4u;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kFewWaves * kWave > kRed ? kFewWaves * kWave : kRed];
    float* const red = (float*)lds;

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t r = lane & 31u, h = lane >> 5;
    uint8_t* const xs = lds + wave * kWave;
    uint8_t* const ws = xs + kXs;

    // tile of this workgroup (feature-major list; XCD x = b % 8 takes the
    // x-th contiguous eighth when the count allows)
    const uint32_t total = tiles_m * tiles_n, b = blockIdx.x;
    const uint32_t L = total % 8u == 0 ? (b % 8u) * (total / 8u) + b / 8u : b;
    const uint32_t tn = L / tiles_m, tm = L % tiles_m;
    const uint32_t m0 = tm * kFT, n0 = tn * kFF;

    constexpr uint32_t xb = XT == kGgmlF32 ? 4u : 2u;
    const uint32_t S = K / (uint32_t)kBK;
    const uint64_t rb = (WT == kGgmlQ8_0) ? (uint64_t)(K / 32u) * 34u : (uint64_t)(K / 256u) * 144u;
    const uint8_t* const Wt = W + (uint64_t)(row_offset + n0) * rb;
    const uint32_t x_rec = (uint32_t)min((uint64_t)M * K * xb, (uint64_t)0xffffffffu);
    const uint32_t w_rec = (uint32_t)min((uint64_t)(N - n0) * rb, (uint64_t)0xffffffffu);
    // Q8_0: the block's quants start at byte 2 (h = 0) or 4 (h = 1) of the
    // read dwords (a byte-permute selector); Q4_K: nibble h of each byte
    const uint32_t sel = WT == kGgmlQ8_0 ? (h ? 0x07060504u : 0x05040302u) : (h ? 0xf0f0f0f0u : 0x0f0f0f0fu);

    f32x16 acc[kFB];
#pragma unroll
    for (uint32_t fb = 0; fb < kFB; fb++) acc[fb] = f32x16{};

    // this wave's stages: wave, wave + 8, ... (n of them); the load after
    // the last one reads nothing (a descriptor of no bytes). The selected
    // counts and offsets go back through readfirstlane: computed (uniform)
    // in vector registers, they made every buffer load a loop over the
    // lanes' values.
    const uint32_t n = S > wave ? (S - wave + kFewWaves - 1u) / kFewWaves : 0u;
    FewLoads<WT, XT> ld;
    auto load = [&](uint32_t i) {
        const bool live = i < n;
        const uint32_t s = __builtin_amdgcn_readfirstlane(live ? wave + kFewWaves * i : 0u);
        const uint32_t xn = __builtin_amdgcn_readfirstlane(live ? x_rec : 0u);
        const uint32_t wn = __builtin_amdgcn_readfirstlane(live ? w_rec : 0u);
        ld.load(make_rsrc(X, xn), make_rsrc(Wt, wn), m0, K, rb, s, lane);
    };
    load(0);
    for (uint32_t i = 0; i < n; i++) {
        // stage i into the wave's region (after the reads of stage i - 1:
        // a wave's LDS accesses run in order), stage i + 1's loads out, then
        // stage i read back and multiplied
        ld.template store<OT>(xs, ws, lane);
        load(i + 1);
        const uint32_t s = wave + kFewWaves * i;
        FewW<WT> wr[kFB];
        FewWop<WT, OT> wo[kFB];
#pragma unroll
        for (uint32_t fb = 0; fb < kFB; fb++) {
            wr[fb].read(ws, 32u * fb + r, h);
            wo[fb].prepare(wr[fb], h, s & 3u);
        }
#pragma unroll
        for (uint32_t t = 0; t < 4; t++) {
            const f16x8 xo = *(const f16x8*)(xs + lds_off(r, 4u * h + t));
#pragma unroll
            for (uint32_t fb = 0; fb < kFB; fb++) acc[fb] = mfma16<OT>(wo[fb].op(wr[fb], t, sel), xo, acc[fb]);
        }
    }
    __syncthreads();  // every wave is done with its staging region

    // the waves' partial tiles through LDS: lane (token r, kh = h) holds
    // features 32 fb + 8 g + 4 h + 0..3
    float* const mine = red + wave * (kFT * kRedLd);
#pragma unroll
    for (uint32_t fb = 0; fb < kFB; fb++)
#pragma unroll
        for (uint32_t g = 0; g < 4; g++)
            *(f32x4*)(mine + r * kRedLd + 32u * fb + 8u * g + 4u * h) =
                f32x4{acc[fb][4 * g], acc[fb][4 * g + 1], acc[fb][4 * g + 2], acc[fb][4 * g + 3]};
    __syncthreads();
    // 16-byte output pieces p = tid, tid + 512 (row p / 24, features
    // 4 (p % 24) .. + 3 of the tile), each summed over the waves in wave order
    constexpr uint32_t kPieces = kFT * kFF / 4u, kPerRow = kFF / 4u;
    for (uint32_t p = tid; p < kPieces; p += kFewWaves * 64u) {
        const uint32_t row = p / kPerRow, col = 4u * (p % kPerRow), m = m0 + row, nn = n0 + col;
        if (m >= M || nn >= N) continue;
        f32x4 v = *(const f32x4*)(red + row * kRedLd + col);
#pragma unroll
        for (uint32_t w = 1; w < kFewWaves; w++) v += *(const f32x4*)(red + w * (kFT * kRedLd) + row * kRedLd + col);
        float* const yp = Y + (uint64_t)m * N + nn;
        if (N % 4u == 0) {
            *(f32x4*)yp = v;  // nn % 4 == 0, nn + 3 < N
        } else {
            yp[0] = v.x;
            if (nn + 1 < N) yp[1] = v.y;
            if (nn + 2 < N) yp[2] = v.z;
            if (nn + 3 < N) yp[3] = v.w;
        }
    }
}

}  // namespace

hipError_t launch_gemm_few(const void* w, uint32_t wtype, const void* x, uint32_t xtype, float* y, uint32_t N,
                           uint32_t K, uint32_t M, uint32_t row_offset, hipStream_t st) {
    if (M == 0 || M > plan::kFewMaxTokens || K % kBK || K == 0) return hipErrorInvalidValue;
    const uint32_t tiles_m = (M + kFT - 1) / kFT, tiles_n = (N + kFF - 1) / kFF;
    const dim3 grid(tiles_m * tiles_n), block(kFewWaves * 64u);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, st, (const uint8_t*)w, x, y, N, K, M, row_offset, tiles_m, tiles_n);
    };
    if (wtype == kGgmlQ8_0) {
        if (xtype == kGgmlF32) go(gemm_q_few<kGgmlQ8_0, kGgmlF32>);
        else if (xtype == kGgmlF16) go(gemm_q_few<kGgmlQ8_0, kGgmlF16>);
        else go(gemm_q_few<kGgmlQ8_0, kGgmlBF16>);
    } else {
        if (xtype == kGgmlF32) go(gemm_q_few<kGgmlQ4K, kGgmlF32>);
        else if (xtype == kGgmlF16) go(gemm_q_few<kGgmlQ4K, kGgmlF16>);
        else go(gemm_q_few<kGgmlQ4K, kGgmlBF16>);
    }
    return hipGetLastError();
}

}  // namespace llmr
