// gemm_w16.hip - the two-pass dequant-GEMM for many tokens.
//
//   Y[m, n] = sum_k X[m, k] * W[row_offset + n, k]     (f32 out)
//
// Same operands and the same MFMA order as the fused persistent kernel
// (gemm_q_persist): the result is bit-identical. What differs is where the
// dequantization happens. The fused kernel dequantizes a weight tile once per
// 256-token tile it multiplies, inside its stage loop, where the VALU work
// and the register staging of the packed bytes compete with the MFMAs of the
// same wave. With thousands of tokens each weight row is dequantized M / 256
// times (18 times at M = 4608). Here:
//   pass 1 (w16_image_kernel) dequantizes every weight element once into a
//          16-bit image of the weight, laid out exactly as the GEMM's LDS
//          tiles: for each 256-row panel and each 64-wide K stage a
//          contiguous 32 KiB block, row r at r * 128 bytes, 16-byte chunk c
//          at (c ^ lds_swz(r)) * 16;
//   pass 2 (gemm_w16_persist) is the persistent 256 x 256 kernel with both
//          operands copied HBM -> LDS by buffer DMA (the weight block is one
//          contiguous 32 KiB copy): a stage is 64 MFMAs, 32 fragment reads
//          and 16 DMAs per wave, no dequantization and no register staging.
// The image costs N * K * 2 bytes of workspace and one write + one read of
// it; the dispatcher takes this path when M is large enough for that to pay.
#include "gemm_q_common.h"
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

constexpr uint32_t kBlk = 256u * 128u;  // bytes of one 256-row x 64-wide 16-bit block

// Pass 1. Workgroup (panel p, stage group j), thread r: weight row r of the
// panel for stages 4j .. 4j+3 (one Q4_K superblock, eight Q8_0 blocks: the
// row's bytes of the group are read by this one thread, so no other
// workgroup - on another XCD, with its own L2 - fetches them again),
// dequantized with the fused kernel's own WRow code (operand type OT: bf16
// for bf16 activations, fp16 otherwise) into a 32 KiB block in LDS, which
// the workgroup then copies to image block (p, s) in 16-byte pieces of
// consecutive addresses (each store instruction writes 1 KiB of whole
// lines; written straight from the rows, every instruction would touch 64
// lines). Two LDS blocks alternate, so one barrier per stage suffices. SW:
// the panel is a 128-feature SwiGLU tile, rows gate 0-63 | up 0-63 | gate
// 64-127 | up 64-127 (the fused SwiGLU kernel's LDS arrangement). Rows past
// N read as zero through the descriptor and give zero operands.
//
// LORA: a LoRA adapter merged into the image (the reference applies it as a
// correction after the GEMM, dispatch_lora_correction): feature n in
// [lro, lro + b_rows) of the panel gets d[n, k] = sum_r (scale b[wro + n -
// lro, r]) a[r, k] added to its dequantized weight in f32, then the 16-bit
// rounding once more (features outside keep their image bit for bit). d is
// a 256 x 64 x rank product per stage, computed on the matrix cores as d^T =
// a^T (scale b)^T with 32x32x16 bf16 MFMAs: both factors split into bf16
// hi + lo parts (x = hi + lo to 2^-17 relative) and summed as hi hi + hi lo
// + lo hi, so d carries about 16 correct bits (the dropped lo lo term is
// 2^-16 of it) - far below the 16-bit rounding that follows. Wave w holds the
// (scale b)^T fragments of panel rows 64 w .. 64 w + 63 in registers for the
// whole workgroup and loads each stage's a^T fragments (f32, from L2) one
// stage ahead; a lane's accumulators are four consecutive k of one of its
// wave's rows, one 8-byte read-modify-write of the LDS block.
constexpr uint32_t kImgStages = 4;
constexpr uint32_t kLoraSteps = kLoraImageMaxRank / 16u;  // 16-wide rank steps
struct ImageLora {
    const float* a;  // [rank, K]
    const float* b;  // [*, rank]
    float scale;
    uint32_t rank, lro, b_rows, wro;
};
// x -> (bf16 hi, bf16 lo) with x = hi + lo to 2^-17 relative, packed for
// eight values into two 16-byte MFMA operands
__device__ __forceinline__ void split_bf16x8(const float (&v)[8], u32x4& hi, u32x4& lo) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (uint32_t e = 0; e < 4; e++) {
        const bf16x2_t h{(__bf16)v[2 * e], (__bf16)v[2 * e + 1]};
        const bf16x2_t l{(__bf16)(v[2 * e] - (float)h[0]), (__bf16)(v[2 * e + 1] - (float)h[1])};
        hi[e] = __builtin_bit_cast(uint32_t, h);
        lo[e] = __builtin_bit_cast(uint32_t, l);
    }
}
// Items (panel p, group of kImgStages stages) of a weight's image:
// panels * groups of them, item = p * groups + group; a panel is 256 rows
// (SwiGLU: 128 outputs, their gate and up rows).
__host__ __device__ __forceinline__ uint32_t image_groups(uint32_t K) {
    return (K / (uint32_t)kBK + kImgStages - 1) / kImgStages;
}
__host__ __device__ __forceinline__ uint32_t image_items(uint32_t N, uint32_t K, bool sw = false) {
    return (sw ? (N + 127u) / 128u : (N + 255u) / 256u) * image_groups(K);
}
// One item of an image without LoRA by the 256 threads of a workgroup
// (thread r: row r of the panel), through the two 32 KiB LDS blocks lb0 and
// lb1 (one barrier per stage), or through one (ONE: lb0 == lb1, a second
// barrier per stage). Callers running several items in a row put a barrier
// between them. Plain (SW false): rows row_offset + 256 p + r of
// W. SW: the SwiGLU arrangement of N outputs, W the gate rows and W2 the up
// rows of output 0 (row_offset unused): panel p holds outputs 128 p .. +
// 127, its rows gate 0-63 | up 0-63 | gate 64-127 | up 64-127 (wave q of
// the workgroup: gate or up by q % 2, outputs 64 (q / 2) ..), the
// arrangement of the fused SwiGLU kernel. NT: non-temporal stores (items
// built beside a running GEMM: streamed, they evict less of its operands
// from L2; Flux step 76.3 -> 75.8 ms).
template <uint32_t WT, uint32_t OT, bool NT = false, bool SW = false, bool ONE = false>
__device__ __forceinline__ void image_item(const uint8_t* __restrict__ W, const uint8_t* __restrict__ W2,
                                           uint8_t* __restrict__ img, uint32_t N, uint32_t K, uint32_t row_offset,
                                           uint32_t item, uint8_t* lb0, uint8_t* lb1) {
    const uint32_t S = K / kBK, groups = image_groups(K);
    const uint32_t p = item / groups, s0 = (item % groups) * kImgStages, r = threadIdx.x;
    const uint32_t rb = (WT == kGgmlQ8_0) ? (K / 32u) * 34u : (K / 256u) * 144u;
    const uint8_t* src;
    uint32_t n0, row;  // the panel's first feature, this thread's row of it
    if constexpr (SW) {
        const uint32_t q = __builtin_amdgcn_readfirstlane(r >> 6);
        n0 = 128u * p;
        src = (q & 1u) ? W2 : W;
        row = (q >> 1) * 64u + (r & 63u);
    } else {
        n0 = 256u * p;
        src = W + (uint64_t)row_offset * rb;
        row = r;
    }
    const rsrc_t rs = make_rsrc(src + (uint64_t)n0 * rb, (uint64_t)(N - n0) * rb);
    WRow<WT, OT> u[kImgStages];
#pragma unroll
    for (uint32_t i = 0; i < kImgStages; i++)
        if (s0 + i < S)
            static_for<0, WRow<WT, OT>::kLoads>(
                [&](auto L) { u[i].template load<decltype(L)::value>(rs, row * rb, s0 + i); });
    const uint32_t base = r * 128u + (lds_swz(r) << 4);
#pragma unroll
    for (uint32_t i = 0; i < kImgStages; i++) {
        if (s0 + i >= S) break;
        uint8_t* const lb = (i & 1u) ? lb1 : lb0;
        const auto sc = u[i].scale(s0 + i);
        u[i].template store<0>(lb, sc, base);
        u[i].template store<1>(lb, sc, base);
        u[i].template store<2>(lb, sc, base);
        u[i].template store<3>(lb, sc, base);
        __syncthreads();
        u32x4* const dst = (u32x4*)(img + ((uint64_t)p * S + s0 + i) * kBlk);
#pragma unroll
        for (uint32_t c = 0; c < kBlk / 16u / 256u; c++) {
            if constexpr (NT)
                __builtin_nontemporal_store(((const u32x4*)lb)[r + 256u * c], dst + r + 256u * c);
            else
                dst[r + 256u * c] = ((const u32x4*)lb)[r + 256u * c];
        }
        if constexpr (ONE)
            if (i + 1u < kImgStages) __syncthreads();  // the block is read out before the next stage's stores
    }
}

template <uint32_t WT, uint32_t OT, bool SW, uint32_t RS = 0>
__global__ void __launch_bounds__(256) w16_image_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ W2,
                                                         uint8_t* __restrict__ img, uint32_t N, uint32_t K,
                                                         uint32_t row_offset, const ImageLora lo, uint32_t item0) {
    if constexpr (RS == 0) {  // no LoRA: item item0 + blockIdx.x, through one 32 KiB block
        __shared__ __attribute__((aligned(16))) uint8_t blk[kBlk];
        image_item<WT, OT, false, SW, true>(W, W2, img, N, K, row_offset, item0 + blockIdx.x, blk, blk);
        return;
    }
    constexpr bool LORA = RS > 0;         // RS: rank steps of 16 the kernel holds (rank <= 16 RS)
    constexpr uint32_t RA = LORA ? RS : 1u;  // register array extent
    // one LDS object: two image blocks, then (LORA) the stage's a^T
    // fragments, [k tile 2][rank step RS][hi, lo][64 lanes] x 16 B; before
    // the first stage the panel's b rows are staged across all of it
    constexpr uint32_t kAfr = LORA ? 2u * RS * 2u * 64u * 16u : 0u;
    __shared__ __attribute__((aligned(16))) uint8_t lds[2u * kBlk + kAfr];
    uint8_t(*const lblk)[kBlk] = (uint8_t(*)[kBlk])lds;
    u32x4* const afr = (u32x4*)(lds + 2u * kBlk);
    const uint32_t S = K / kBK, groups = (S + kImgStages - 1) / kImgStages;
    const uint32_t p = blockIdx.x / groups, s0 = (blockIdx.x % groups) * kImgStages, r = threadIdx.x;
    const uint32_t rb = (WT == kGgmlQ8_0) ? (K / 32u) * 34u : (K / 256u) * 144u;
    const uint8_t* src;
    uint32_t n0, row;  // first feature of the panel, this thread's row within it
    if constexpr (SW) {
        n0 = 128u * p;
        const uint32_t q = r >> 6;
        src = (q & 1u) ? W2 : W;
        row = (q >> 1) * 64u + (r & 63u);
    } else {
        n0 = 256u * p;
        src = W + (uint64_t)row_offset * rb;
        row = r;
    }
    // LORA loads go first, ahead of the weight rows: they are L2 hits and
    // return before the rows, so waiting for them (the memory counter is in
    // order) costs nothing the rows do not.
    //  bv: the panel's b rows, element u = r + 256 i of [256 rows][16 RS]
    //      (consecutive threads read consecutive floats of a row);
    //  av: a for the thread's units q = r + 256 h of each stage (rank group
    //      rg = q / 64, column k = q % 64, rows 8 rg .. 8 rg + 7).
    // Rows outside the slot and ranks >= rank lie past the descriptors'
    // ranges and read as zero, so every load is unconditional.
    const uint32_t wave = r >> 6, lane = r & 63u;
    float bv[LORA ? RS * 16u : 1u], av[kImgStages][LORA ? RS / 2u : 1u][8];
    bool in_slot[2] = {false, false};
    bool wave_any = false;
    if constexpr (LORA) {
        const rsrc_t rbv = make_rsrc(lo.b + (uint64_t)lo.wro * lo.rank, (uint64_t)lo.b_rows * lo.rank * 4u);
#pragma unroll
        for (uint32_t i = 0; i < RS * 16u; i++) {
            const uint32_t u = r + 256u * i, n = n0 + u / (16u * RS), c = u % (16u * RS);
            const bool ok = n < N && n >= lo.lro && n - lo.lro < lo.b_rows && c < lo.rank;
            bv[i] = __uint_as_float(bload4(rbv, ok ? ((n - lo.lro) * lo.rank + c) * 4u : ~0u, 0u));
        }
        const rsrc_t rav = make_rsrc(lo.a, (uint64_t)lo.rank * K * 4u);
#pragma unroll
        for (uint32_t i = 0; i < kImgStages; i++)
#pragma unroll
            for (uint32_t h = 0; h < RS / 2u; h++) {
                const uint32_t q = r + 256u * h, k = q & 63u, rg = q >> 6;
                const uint32_t st = min(s0 + i, S - 1u);
#pragma unroll
                for (uint32_t e = 0; e < 8; e++)
                    av[i][h][e] = __uint_as_float(bload4(rav, ((8u * rg + e) * K + 64u * st + k) * 4u, 0u));
            }
    }
    const rsrc_t rs = make_rsrc(src + (uint64_t)n0 * rb, (uint64_t)(N - n0) * rb);
    WRow<WT, OT> u[kImgStages];
#pragma unroll
    for (uint32_t i = 0; i < kImgStages; i++)
        if (s0 + i < S)
            static_for<0, WRow<WT, OT>::kLoads>(
                [&](auto L) { u[i].template load<decltype(L)::value>(rs, row * rb, s0 + i); });
    const uint32_t base = r * 128u + (lds_swz(r) << 4);
    // LORA: the wave's (scale b)^T MFMA fragments, rows 64 wave + 32 nt +
    // l32 and ranks 16 j + 8 kh + 0..7, through LDS (row stride 16 RS + 4
    // floats: the 16-byte fragment reads of 32 rows fall in distinct banks)
    u32x4 bh[2][RA], bl[2][RA];
    if constexpr (LORA) {
        constexpr uint32_t ld = 16u * RS + 4u;
        float* const bs = (float*)lds;
#pragma unroll
        for (uint32_t i = 0; i < RS * 16u; i++) {
            const uint32_t u = r + 256u * i;
            bs[(u / (16u * RS)) * ld + u % (16u * RS)] = bv[i];
        }
        __syncthreads();
        const uint32_t w0 = n0 + 64u * wave;  // the wave's rows [w0, w0 + 64) of the weight
        wave_any = w0 < N && w0 + 64u > lo.lro && w0 < lo.lro + lo.b_rows;
#pragma unroll
        for (uint32_t nt = 0; nt < 2; nt++) {
            const uint32_t pr = 64u * wave + 32u * nt + (lane & 31u), n = n0 + pr;
            in_slot[nt] = n < N && n >= lo.lro && n - lo.lro < lo.b_rows;
#pragma unroll
            for (uint32_t j = 0; j < RS; j++) {
                const float* const src8 = bs + pr * ld + 16u * j + 8u * (lane >> 5);
                const f32x4 x0 = *(const f32x4*)src8, x1 = *(const f32x4*)(src8 + 4);
                const float v[8] = {lo.scale * x0[0], lo.scale * x0[1], lo.scale * x0[2], lo.scale * x0[3],
                                    lo.scale * x1[0], lo.scale * x1[1], lo.scale * x1[2], lo.scale * x1[3]};
                split_bf16x8(v, bh[nt][j], bl[nt][j]);
            }
        }
        __syncthreads();  // the staged b is read before the first stage's stores
    }
#pragma unroll
    for (uint32_t i = 0; i < kImgStages; i++) {
        if (s0 + i >= S) break;
        uint8_t* const lb = lblk[i & 1u];
        const auto sc = u[i].scale(s0 + i);
        u[i].template store<0>(lb, sc, base);
        u[i].template store<1>(lb, sc, base);
        u[i].template store<2>(lb, sc, base);
        u[i].template store<3>(lb, sc, base);
        if constexpr (LORA) {
            // the stage's a split into its MFMA fragments in afr
#pragma unroll
            for (uint32_t h = 0; h < RS / 2u; h++) {
                const uint32_t q = r + 256u * h, k = q & 63u, rg = q >> 6;
                const uint32_t slot = ((k >> 5) * RS + (rg >> 1)) * 128u + 32u * (rg & 1u) + (k & 31u);
                split_bf16x8(av[i][h], afr[slot], afr[slot + 64u]);
            }
            __syncthreads();
            if (wave_any) {
#pragma unroll
                for (uint32_t t = 0; t < 2; t++) {
                    f32x16 acc[2] = {f32x16{}, f32x16{}};
#pragma unroll
                    for (uint32_t j = 0; j < RS; j++) {
                        const u32x4 ah = afr[(t * RS + j) * 128u + lane];
                        const u32x4 alo = afr[(t * RS + j) * 128u + 64u + lane];
#pragma unroll
                        for (uint32_t nt = 0; nt < 2; nt++) {
                            acc[nt] = mfma16<kGgmlBF16>(__builtin_bit_cast(f16x8, ah),
                                                        __builtin_bit_cast(f16x8, bh[nt][j]), acc[nt]);
                            acc[nt] = mfma16<kGgmlBF16>(__builtin_bit_cast(f16x8, ah),
                                                        __builtin_bit_cast(f16x8, bl[nt][j]), acc[nt]);
                            acc[nt] = mfma16<kGgmlBF16>(__builtin_bit_cast(f16x8, alo),
                                                        __builtin_bit_cast(f16x8, bh[nt][j]), acc[nt]);
                        }
                    }
                    // lane: row 64 w + 32 nt + l32, k = 32 t + 8 g + 4 kh + 0..3
#pragma unroll
                    for (uint32_t nt = 0; nt < 2; nt++) {
                        if (!in_slot[nt]) continue;
                        const uint32_t pr = 64u * wave + 32u * nt + (lane & 31u);
#pragma unroll
                        for (uint32_t g = 0; g < 4; g++) {
                            u32x2* const cell =
                                (u32x2*)(lb + pr * 128u + (((4u * t + g) ^ lds_swz(pr)) << 4) + 8u * (lane >> 5));
                            u32x2 v = *cell;
#pragma unroll
                            for (uint32_t e = 0; e < 2; e++) {
                                const float d0 = acc[nt][4 * g + 2 * e], d1 = acc[nt][4 * g + 2 * e + 1];
                                if constexpr (OT == kGgmlBF16) {
                                    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
                                    v[e] = __builtin_bit_cast(
                                        uint32_t, bf16x2_t{(__bf16)(__uint_as_float(v[e] << 16) + d0),
                                                           (__bf16)(__uint_as_float(v[e] & 0xffff0000u) + d1)});
                                } else {
                                    v[e] = pack_f16x2(
                                        (float)__builtin_bit_cast(_Float16, (uint16_t)(v[e] & 0xffffu)) + d0,
                                        (float)__builtin_bit_cast(_Float16, (uint16_t)(v[e] >> 16)) + d1);
                                }
                            }
                            *cell = v;
                        }
                    }
                }
            }
        }
        __syncthreads();
        u32x4* const dst = (u32x4*)(img + ((uint64_t)p * S + s0 + i) * kBlk);
#pragma unroll
        for (uint32_t c = 0; c < kBlk / 16u / 256u; c++) dst[r + 256u * c] = ((const u32x4*)lb)[r + 256u * c];
    }
}

// Plain-store epilogue of gemm_w16_persist through LDS. The
// accumulators hold, per lane, 16-byte pieces of one token row (lane l32:
// token 32 b + l32, features 32 a + 8 g + 4 kh + 0..3), so stored as they
// are every store instruction writes 32-byte pieces of 32 rows. Here a wave
// stages 32 token rows x 64 features at a time (acc[a][b] for two a) in 8
// KiB of LDS (row r at r * 256 bytes, 16-byte chunk c at (c ^ (r % 16)) *
// 16) and stores four whole 256-byte row segments per instruction. `st` is
// the wave's own quarter of a ring slot the tile's last stage read: only
// this wave's DMAs of the next stage overwrite it, issued after this, and a
// wave's LDS accesses run in order (no barrier). One LDS object, so the
// compiler does not wait for the DMAs in flight into the other slots.
// Measured on one box: flux_linear1 0.562 -> 0.554 ms, zimage_qkv 0.394 ->
// 0.389 ms. The gated-residual epilogue staged the same way made the Flux
// step 1% slower (its loads of the residual rows dominate), and the
// split-gelu one's per-lane choice of side made the compiler treat the load
// cursors as divergent: both keep the direct stores.
// The stores are non-temporal (streamed through L2: a tile's 256 KiB of
// results are not read again by this kernel, its operand panels are; the L2
// hit rates were not counted): flux_linear1 0.583 -> 0.568 ms,
// flux_linear2 0.440 -> 0.423 ms, the Flux step 79.1 -> 78.9 ms (three
// runs each). The gated-residual and split-gelu
// epilogues keep cached stores: streamed, their rows (read again by the
// next block's glue) made the step 0.7% slower.
__device__ __forceinline__ void store_tile_rows(f32x16 (&acc)[4][4], float* Y, uint32_t M, uint32_t N, uint32_t m0,
                                                uint32_t n0, uint32_t wm, uint32_t wn, uint32_t lane, uint32_t ldy,
                                                uint8_t* st) {
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const uint32_t c = lane & 15u, rq = lane >> 4;  // read back: chunk c of row 4 i + rq
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t n = n0 + wn * 128u + 64u * h + 4u * c;
#pragma unroll
        for (int b = 0; b < 4; b++) {
#pragma unroll
            for (int a = 2 * h; a < 2 * h + 2; a++) {
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *(f32x4*)(st + l32 * 256u + (((8u * (a - 2 * h) + 2u * g + kh) ^ (l32 & 15u)) << 4)) =
                        f32x4{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
                acc[a][b] = f32x16{};
            }
            f32x4 v[8];  // all eight reads before the stores
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t r = 4u * i + rq;
                v[i] = *(const f32x4*)(st + r * 256u + ((c ^ (r & 15u)) << 4));
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t m = m0 + wm * 128u + 32u * b + 4u * i + rq;
                if (m < M && n < N) __builtin_nontemporal_store(v[i], (f32x4*)(Y + (uint64_t)m * ldy + n));
            }
        }
    }
}

// One 16-wide k step of the all-DMA stage: 16 MFMAs, the next step's eight
// fragment reads after the first eight, the step's four DMAs after the next
// four.
#define LLMR16_STEP_SCHEDULE                                                                   \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1);           \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1);           \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1);           \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1); LLMR_SGB(0x008, 1); LLMR_SGB(0x100, 1);           \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x020, 1); LLMR_SGB(0x008, 1); LLMR_SGB(0x020, 1);           \
    LLMR_SGB(0x008, 1); LLMR_SGB(0x020, 1); LLMR_SGB(0x008, 1); LLMR_SGB(0x020, 1);           \
    LLMR_SGB(0x008, 4)

// Pass 2: the persistent 256 x 256 kernel (tile order, wave layout,
// fragment reads, MFMA order and epilogues of gemm_q_persist) with the weight
// operand DMA'd from the image. LDS: five 32 KiB slots, three for the
// activations (fetched two stages ahead) and two for the weights (one stage
// ahead: the image blocks are contiguous, and each is shared by the four
// tile rows an XCD runs at once).
//   args.p[i].W  the image of problem i (block (panel, stage) at
//                (panel * K/64 + stage) * 32 KiB); row_offset is unused (the
//                image starts at the problem's first feature).
template <uint32_t XT, bool SW, uint32_t EPI = kEpiStore, bool GROUPED = false>
__global__ void __launch_bounds__(256, 1) gemm_w16_persist(const PersistArgs args) {
    static_assert(!(SW && GROUPED) && (!SW || EPI == kEpiStore), "SwiGLU launches are single, plain stores");
    static_assert(XT == kGgmlF16 || XT == kGgmlBF16, "16-bit activations only");
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
    const uint32_t Tp0 = args.p[0].tiles_m;
    constexpr uint32_t NT = SW ? 128u : 256u;  // output features per tile
    constexpr int DMAS = 8;                    // 1 KiB DMAs per wave per operand per stage
    __shared__ __attribute__((aligned(16))) uint8_t X0[kBlk];
    __shared__ __attribute__((aligned(16))) uint8_t X1[kBlk];
    __shared__ __attribute__((aligned(16))) uint8_t X2[kBlk];
    __shared__ __attribute__((aligned(16))) uint8_t W0[kBlk];
    __shared__ __attribute__((aligned(16))) uint8_t W1[kBlk];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const uint32_t wm = wave & 1u, wn = wave >> 1;

    const uint32_t G = gridDim.x, total = tiles_m * tiles_n;
    const uint32_t n_tiles = w16_n_tiles(blockIdx.x, G, total);  // 0: no tile (grid = the CUs > total)
    const uint32_t S = K / kBK;
    const uint32_t SP = (S + 5u) / 6u * 6u;
    const uint32_t xrow = K * 2u;
    const uint32_t panel = S * kBlk;  // image bytes of one 256-row panel

    // activation DMA i of wave w: rows 64w + 8i + lane/8, physical chunk
    // lane%8, logical chunk (lane%8) ^ lds_swz(row); weight DMA i of wave w:
    // bytes 8192 w + 1024 i + 16 lane of the block, copied as they are
    uint32_t xvoff[DMAS];
#pragma unroll
    for (int i = 0; i < DMAS; i++) {
        const uint32_t row = 64u * wave + 8u * i + (lane >> 3);
        const uint32_t c = (lane & 7u) ^ lds_swz(row);
        xvoff[i] = row * xrow + c * 16u;
    }
    const uint32_t wvoff = wave * 8192u + lane * 16u;
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t ch = 4u * (t >> 1) + 2u * kh + (t & 1);
        xoff[t] = lds_off(wm * 128u + l32, ch);
        woff[t] = lds_off(wn * 128u + l32, ch);
    }

    struct Cursor {
        uint32_t s;               // stage within the tile
        const uint8_t* base;      // the tile's first activation row / its image panel
        uint32_t size;            // bytes readable from base (0 past the last tile)
    };
    auto tile_origin = [&](uint32_t k, uint32_t& p, uint32_t& m0, uint32_t& n0) {
        uint32_t tm, tn;
        w16_tile(blockIdx.x, k, G, tiles_m, tiles_n, tm, tn);
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
        c.base = pick(p, Wp0, Wp1) + (uint64_t)(n0 / NT) * panel;
        c.size = k < n_tiles ? panel : 0u;
    };
    Cursor cx{0, nullptr, 0}, cw{0, nullptr, 0};
    Cursor nx{0, nullptr, 0}, nw{0, nullptr, 0};
    auto advance = [&](Cursor& c, const Cursor& next) {
        if (++c.s == SP) c = next;
    };
    auto xdma = [&](rsrc_t xr, uint8_t* Xs, int i, uint32_t so) {
        uint8_t* dst = Xs + wave * (64u * 128u) + 1024u * i;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)dst, 16, xvoff[i], so, 0, 0);
    };
    auto wdma = [&](rsrc_t wr, uint8_t* Ws, int i, uint32_t so) {
        uint8_t* dst = Ws + wave * 8192u + 1024u * i;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)dst, 16, wvoff + 1024u * i, so, 0, 0);
    };
    auto x_rsrc = [&]() { return make_rsrc(cx.base, cx.s < S ? cx.size : 0u); };
    auto w_rsrc = [&]() { return make_rsrc(cw.base, cw.s < S ? cw.size : 0u); };
    // part p of a stage's loads: the weights of the next stage (parts 0-1),
    // then the activations two stages ahead (parts 2-3)
    auto issue_part = [&](auto PART, rsrc_t wr, uint32_t wso, uint8_t* Wd, rsrc_t xr, uint32_t xso, uint8_t* Xd) {
        constexpr int p = decltype(PART)::value;
        static_for<4 * p, 4 * p + 4>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if constexpr (i < DMAS)
                wdma(wr, Wd, i, wso);
            else
                xdma(xr, Xd, i - DMAS, xso);
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
    // after a tile's last stage (the loop's sixth, which read X2 and W1)
    auto store_tile = [&](uint32_t k) {
        uint32_t p, m0, n0;
        tile_origin(k, p, m0, n0);
        if constexpr (!SW && EPI == kEpiStore)
            store_tile_rows(acc, pick(p, Yp0, Yp1), pick(p, Mp0, Mp1), N, m0, n0, wm, wn, lane, ldy,
                            X2 + wave * 8192u);
        else
            store_tile_256<SW, EPI, true>(acc, pick(p, Yp0, Yp1), pick(p, Gp0, Gp1), pick(p, Y2p0, Y2p1),
                                          pick(p, Mp0, Mp1), N, m0, n0, wm, wn, l32, kh, ldy, ldy2, split, y2_bf16,
                                          &args.heads, p, X2 + wave * 8192u, W1 + wave * 8192u);
    };

    if (n_tiles > 0) {
    // prologue: W(0) -> W0, X(0) -> X0, X(1) -> X1 (in the steady state's
    // order: a stage issues W(g+1), then X(g+2)); stage 0's operands have
    // landed once at most X(1)'s DMAs are in flight
    x_tile(cx, 0);
    w_tile(cw, 0);
    x_tile(nx, 1);
    w_tile(nw, 1);
    {
        const rsrc_t wr = w_rsrc();
#pragma unroll
        for (int i = 0; i < DMAS; i++) wdma(wr, W0, i, cw.s * kBlk);
        advance(cw, nw);
        const rsrc_t xr = x_rsrc();
#pragma unroll
        for (int i = 0; i < DMAS; i++) xdma(xr, X0, i, cx.s * 128u);
        advance(cx, nx);
        const rsrc_t xr1 = x_rsrc();
#pragma unroll
        for (int i = 0; i < DMAS; i++) xdma(xr1, X1, i, cx.s * 128u);
        advance(cx, nx);
    }
    LLMR_STAGE_BARRIER(DMAS);

    Frags F0, F1;

    // Global stage g reads X[g%3], W[g%2] and issues W(g+1) -> W[(g+1)%2] and
    // X(g+2) -> X[(g+2)%3] (both slots were last read in stage g-1, before
    // the previous barrier). The barrier at its end waits until at most
    // X(g+2)'s DMAs are in flight: W(g+1) and X(g+1) have landed.
#define LLMR16_STAGE(XC, WC, XD, WD)                                                          \
    {                                                                                       \
        const rsrc_t wr_ = w_rsrc();                                                        \
        const rsrc_t xr_ = x_rsrc();                                                        \
        const uint32_t wso_ = cw.s * kBlk, xso_ = cx.s * 128u;                              \
        issue_part(std::integral_constant<int, 0>{}, wr_, wso_, WD, xr_, xso_, XD);          \
        read_frags(F0, XC, WC, 0);                                                          \
        mfma_step(F1);                                                                      \
        LLMR16_STEP_SCHEDULE;                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 1>{}, wr_, wso_, WD, xr_, xso_, XD);          \
        read_frags(F1, XC, WC, 1);                                                          \
        mfma_step(F0);                                                                      \
        LLMR16_STEP_SCHEDULE;                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 2>{}, wr_, wso_, WD, xr_, xso_, XD);          \
        read_frags(F0, XC, WC, 2);                                                          \
        mfma_step(F1);                                                                      \
        LLMR16_STEP_SCHEDULE;                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        issue_part(std::integral_constant<int, 3>{}, wr_, wso_, WD, xr_, xso_, XD);          \
        read_frags(F1, XC, WC, 3);                                                          \
        mfma_step(F0);                                                                      \
        LLMR16_STEP_SCHEDULE;                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                  \
        advance(cw, nw);                                                                    \
        advance(cx, nx);                                                                    \
        LLMR_STAGE_BARRIER(DMAS);                                                           \
    }
    for (uint32_t k = 0; k < n_tiles; k++) {
        if (k > 0) {  // the load cursors have moved on to tile k: prepare tile k+1
            x_tile(nx, k + 1);
            w_tile(nw, k + 1);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            F1.x[i] = f16x8{};
            F1.w[i] = f16x8{};
        }
        for (uint32_t s0 = 0; s0 < SP; s0 += 6) {
            LLMR16_STAGE(X0, W0, X2, W1)
            LLMR16_STAGE(X1, W1, X0, W0)
            LLMR16_STAGE(X2, W0, X1, W1)
            LLMR16_STAGE(X0, W1, X2, W0)
            LLMR16_STAGE(X1, W0, X0, W1)
            LLMR16_STAGE(X2, W1, X1, W0)
        }
        mfma_step(F1);
        store_tile(k);
    }
#undef LLMR16_STAGE
    }

    // Later groups' weight images: the workgroups without a tile in the
    // last round build items [0, next.items) between them, through the
    // first two ring slots (no DMA in flight into them after this wait).
    const NextImages& ni = args.next;
    if (ni.items > 0 && total % G != 0 && n_tiles == total / G) {
        LLMR_WAIT_VMCNT(0);
        __syncthreads();
        const uint32_t idle = G - total % G;
        for (uint32_t j = w16_idle_rank(blockIdx.x, G, total); j < ni.items; j += idle) {
            uint32_t i = 0;  // the image of item j (uniform)
            while (i + 1u < ni.count && j >= ni.first[i + 1u]) i++;
            const uint32_t u = j - ni.first[i];
            if (ni.W2[i] == nullptr) {
                if (ni.wtype == kGgmlQ4K)
                    image_item<kGgmlQ4K, XT, true>(ni.W[i], nullptr, ni.img[i], ni.N[i], ni.K[i], ni.row_offset[i],
                                                   u, X0, X1);
                else
                    image_item<kGgmlQ8_0, XT, true>(ni.W[i], nullptr, ni.img[i], ni.N[i], ni.K[i],
                                                    ni.row_offset[i], u, X0, X1);
            } else if (ni.wtype == kGgmlQ4K) {
                image_item<kGgmlQ4K, XT, true, true>(ni.W[i], ni.W2[i], ni.img[i], ni.N[i], ni.K[i], 0u, u, X0, X1);
            } else {
                image_item<kGgmlQ8_0, XT, true, true>(ni.W[i], ni.W2[i], ni.img[i], ni.N[i], ni.K[i], 0u, u, X0, X1);
            }
            __syncthreads();
        }
    }
    LLMR_WAIT_VMCNT(0);  // no DMA may still be writing this workgroup's LDS when it exits
}

// The image's items [item0, all) (item0 > 0 only without LoRA).
template <uint32_t WT, uint32_t OT, bool SW, uint32_t RS = 0>
hipError_t build_image(const void* w, const void* w2, void* img, uint32_t N, uint32_t K, uint32_t row_offset,
                       hipStream_t st, const ImageLora& lo = ImageLora{}, uint32_t item0 = 0) {
    const uint32_t panels = SW ? (N + 127u) / 128u : (N + 255u) / 256u;
    const uint32_t blocks = panels * image_groups(K);
    if (item0 >= blocks) return hipSuccess;
    hipLaunchKernelGGL((w16_image_kernel<WT, OT, SW, RS>), dim3(blocks - item0), dim3(256), 0, st, (const uint8_t*)w,
                       (const uint8_t*)w2, (uint8_t*)img, N, K, row_offset, lo, item0);
    return hipGetLastError();
}

// One workgroup per CU, also when there are fewer tiles (the workgroups
// without one build the next group's images, or end at once).
template <uint32_t XT, bool SW, uint32_t EPI, bool GROUPED>
hipError_t launch_w16(const PersistArgs& a, int num_cus, hipStream_t st) {
    const uint32_t grid = (uint32_t)num_cus;
    hipLaunchKernelGGL((gemm_w16_persist<XT, SW, EPI, GROUPED>), dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <uint32_t XT>
hipError_t launch_w16_epi(const PersistArgs& a, bool grouped, int num_cus, hipStream_t st) {
    switch (a.epi) {
        case kEpiResidual:
            return grouped ? launch_w16<XT, false, kEpiResidual, true>(a, num_cus, st)
                           : launch_w16<XT, false, kEpiResidual, false>(a, num_cus, st);
        case kEpiSplitGelu:
            return grouped ? launch_w16<XT, false, kEpiSplitGelu, true>(a, num_cus, st)
                           : launch_w16<XT, false, kEpiSplitGelu, false>(a, num_cus, st);
        case kEpiSplitSwiglu:
            return grouped ? launch_w16<XT, false, kEpiSplitSwiglu, true>(a, num_cus, st)
                           : launch_w16<XT, false, kEpiSplitSwiglu, false>(a, num_cus, st);
        default:
            return grouped ? launch_w16<XT, false, kEpiStore, true>(a, num_cus, st)
                           : launch_w16<XT, false, kEpiStore, false>(a, num_cus, st);
    }
}

}  // namespace

hipError_t launch_w16_image(const void* w, const void* w2, uint32_t wtype, uint32_t otype, void* img, uint32_t N,
                            uint32_t K, uint32_t row_offset, hipStream_t st, uint32_t item0) {
    const bool sw = w2 != nullptr;
    const ImageLora no{};
    if (wtype == kGgmlQ8_0) {
        if (otype == kGgmlBF16)
            return sw ? build_image<kGgmlQ8_0, kGgmlBF16, true>(w, w2, img, N, K, row_offset, st, no, item0)
                      : build_image<kGgmlQ8_0, kGgmlBF16, false>(w, w2, img, N, K, row_offset, st, no, item0);
        return sw ? build_image<kGgmlQ8_0, kGgmlF16, true>(w, w2, img, N, K, row_offset, st, no, item0)
                  : build_image<kGgmlQ8_0, kGgmlF16, false>(w, w2, img, N, K, row_offset, st, no, item0);
    }
    if (sw)
        return otype == kGgmlBF16 ? build_image<kGgmlQ4K, kGgmlBF16, true>(w, w2, img, N, K, row_offset, st, no, item0)
                                  : build_image<kGgmlQ4K, kGgmlF16, true>(w, w2, img, N, K, row_offset, st, no, item0);
    if (otype == kGgmlBF16)
        return build_image<kGgmlQ4K, kGgmlBF16, false>(w, w2, img, N, K, row_offset, st, no, item0);
    return build_image<kGgmlQ4K, kGgmlF16, false>(w, w2, img, N, K, row_offset, st, no, item0);
}

uint32_t w16_image_items(uint32_t N, uint32_t K, bool sw) { return image_items(N, K, sw); }

hipError_t launch_w16_image_lora(const void* w, uint32_t wtype, uint32_t otype, void* img, uint32_t N, uint32_t K,
                                 uint32_t row_offset, const LoraGemm& l, hipStream_t st) {
    if (l.rank == 0 || l.rank > kLoraImageMaxRank) return hipErrorInvalidValue;
    const ImageLora lo{l.a, l.b, l.scale, l.rank, l.row_offset, l.b_rows, l.weight_row_offset};
    auto go = [&](auto rs) {
        constexpr uint32_t R = decltype(rs)::value;
        if (wtype == kGgmlQ8_0)
            return otype == kGgmlBF16
                       ? build_image<kGgmlQ8_0, kGgmlBF16, false, R>(w, nullptr, img, N, K, row_offset, st, lo)
                       : build_image<kGgmlQ8_0, kGgmlF16, false, R>(w, nullptr, img, N, K, row_offset, st, lo);
        return otype == kGgmlBF16 ? build_image<kGgmlQ4K, kGgmlBF16, false, R>(w, nullptr, img, N, K, row_offset, st, lo)
                                  : build_image<kGgmlQ4K, kGgmlF16, false, R>(w, nullptr, img, N, K, row_offset, st, lo);
    };
    // rank <= 32: two rank steps of 16 (fewer registers), else four
    return l.rank <= 32u ? go(std::integral_constant<uint32_t, 2>{}) : go(std::integral_constant<uint32_t, kLoraSteps>{});
}

hipError_t launch_w16_gemm(const PersistArgs& a, uint32_t xtype, bool swiglu, bool grouped, int num_cus,
                           hipStream_t st) {
    if (swiglu)
        return xtype == kGgmlF16 ? launch_w16<kGgmlF16, true, kEpiStore, false>(a, num_cus, st)
                                 : launch_w16<kGgmlBF16, true, kEpiStore, false>(a, num_cus, st);
    return xtype == kGgmlF16 ? launch_w16_epi<kGgmlF16>(a, grouped, num_cus, st)
                             : launch_w16_epi<kGgmlBF16>(a, grouped, num_cus, st);
}

}  // namespace llmr
