// gemm_plan.h - how one dequant-GEMM call is run: which kernel takes it, how
// K is split, which 16-bit operand type f32 activations are rounded to, and
// the workspace layout. Host code only (no HIP types), so the CPU tests can
// sweep shapes through it (tests/c/plan_check.cpp).
//
// Shapes are in GEMM form: M tokens, N output features, K input features
// (BatchMatMulPC's seq_len, out_dim, in_dim, dit.c3:172-178).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <algorithm>

#include "llmr_hip.h"

namespace llmr {
namespace plan {

constexpr uint32_t kF32 = LLMR_GGML_F32, kF16 = LLMR_GGML_F16, kBF16 = LLMR_GGML_BF16;
constexpr uint32_t kQ8_0 = LLMR_GGML_Q8_0, kQ4K = LLMR_GGML_Q4_K;

constexpr uint32_t kStageK = 64;          // K per stage of every MFMA kernel
constexpr uint32_t kImageBlock = 256u * 128u;  // bytes of one 256-row x 64-wide 16-bit image block
// Q4_K weights times at most this many tokens run on the GEMV kernel (an
// HBM-bound weight stream, gemv_q.hip).
constexpr uint32_t kGemvMaxTokens = 4;
// From this many tokens the weight is dequantized once per call into a
// 16-bit image (gemm_w16.hip) instead of once per 256-token tile.
constexpr uint32_t kW16MinTokens = 2048;
// The tiled kernel splits K when it has fewer than kSplitWgsPerCu
// workgroups per CU, with at least kSplitMinStages stages per split.
constexpr uint32_t kSplitWgsPerCu = 2, kSplitMinStages = 4;
// The few-token kernel (gemm_few.hip): a workgroup owns 32 tokens x
// kFewFeatures features over the whole K.
constexpr uint32_t kFewTokens = 32, kFewFeatures = 96, kFewMaxTokens = 256;

inline uint64_t row_bytes_of(uint32_t wtype, uint32_t K) {
    return wtype == kQ8_0 ? (uint64_t)(K / 32) * 34 : (uint64_t)(K / 256) * 144;
}

inline size_t align256(size_t b) { return (b + 255u) / 256u * 256u; }

// The MFMA operand type f32 activations are rounded to. Q8_0: fp16, the
// reference's float16_t(x) of batch_matmul_q8 (llm.slang:1673). Q4_K: bf16
// (batch_matmul_q4k multiplies x in f32, llm.slang:2300-2304, so a value
// beyond fp16's 65504 stays finite there; bf16 keeps f32's range).
inline uint32_t f32_operand_type(uint32_t wtype) { return wtype == kQ4K ? kBF16 : kF16; }

// The MFMA operand type of activations of type xtype against wtype weights.
inline uint32_t operand_type(uint32_t wtype, uint32_t xtype) {
    return xtype == kF32 ? f32_operand_type(wtype) : xtype;
}

// Bytes of the 16-bit weight image of N features (SwiGLU: 128-feature
// panels of gate and up rows) for the two-pass path.
inline size_t w16_image_bytes(uint32_t N, uint32_t K, bool swiglu) {
    const uint64_t panels = swiglu ? (N + 127u) / 128u : (N + 255u) / 256u;
    return (size_t)(panels * (K / kStageK) * kImageBlock);
}

// The split count for `want` splits of S stages such that every split of
// ceil(S / splits) stages is non-empty (the kernels take split z as stages
// [z per, min(S, (z + 1) per)), per = ceil(S / splits)).
inline uint32_t nonempty_splits(uint32_t S, uint32_t want) {
    if (S == 0) return 1;
    uint32_t splits = std::max<uint32_t>(1u, std::min(want, S));
    for (;;) {
        const uint32_t per = (S + splits - 1) / splits, used = (S + per - 1) / per;
        if (used == splits) return splits;
        splits = used;
    }
}

// Whether `splits` splits of S stages are all non-empty (the launchers'
// check before a split launch).
inline bool splits_nonempty(uint32_t S, uint32_t splits) {
    if (splits == 0 || splits > S) return false;
    const uint32_t per = (S + splits - 1) / splits;
    return (S + per - 1) / per == splits;
}

// Bytes of f32 activations rounded to 16 bits for the few-token skinny
// kernel (stage-major); 16-bit activations are read in place.
inline size_t skinny_x_bytes(uint32_t xtype, uint32_t M, uint32_t K) {
    return xtype == kF32 ? align256((size_t)M * K * 2u) : 0u;
}

// The 4-wave tiled kernel's tile (64, 128 or 256 square) and K splits: the
// largest tile that still gives every CU ~1.5 workgroups; launches with fewer
// workgroups than kSplitWgsPerCu per CU split K (at least kSplitMinStages
// stages per split, M * N % 4 == 0 for the reduction).
struct TilePlan {
    uint32_t bm, splits;
};
inline TilePlan plan_tiles(uint32_t wtype, uint32_t N, uint32_t K, uint32_t M, int num_cus) {
    auto wgs = [&](uint32_t bm) { return (uint64_t)((M + bm - 1) / bm) * ((N + bm - 1) / bm); };
    const uint64_t want = (uint64_t)num_cus * 3 / 2;
    TilePlan t{64, 1};
    if (wgs(256) >= want) t.bm = 256;
    else if (wgs(128) >= want) t.bm = 128;
    if (wtype == kQ8_0 && K % kStageK) return t;  // the generic kernel
    const uint64_t w = wgs(t.bm), target = (uint64_t)num_cus * kSplitWgsPerCu;
    const uint32_t S = K / kStageK;
    if (w < target && S >= 2 * kSplitMinStages && ((uint64_t)M * N) % 4 == 0)
        t.splits = nonempty_splits(S, (uint32_t)std::min<uint64_t>((target + w - 1) / w, S / kSplitMinStages));
    return t;
}

// Whether the few-token kernel takes M x N x K: at most kFewMaxTokens
// tokens, whole stages, and at least half the CUs' worth of 32 x 96 tiles
// (fewer: the skinny kernel, which splits K to fill the CUs).
inline bool few_fits(uint32_t N, uint32_t K, uint32_t M, int num_cus) {
    if (M == 0 || M > kFewMaxTokens || K % kStageK || K == 0) return false;
    // 32-bit buffer offsets of the f32 activation rows and of the weight
    // rows past N that a last tile addresses
    if ((uint64_t)(M + kFewTokens) * K * 4u >= (1ull << 31)) return false;
    const uint64_t tiles = (uint64_t)((M + kFewTokens - 1) / kFewTokens) * ((N + kFewFeatures - 1) / kFewFeatures);
    return 2 * tiles >= (uint64_t)num_cus;
}

// How one GEMM runs.
//  * few: the few-token kernel (f32 / 16-bit activations read in place, no
//    workspace);
//  * skinny: the few-token kernel with K splits (M <= 256 with too few 32 x
//    96 tiles): workspace = [f32 activations as 16 bits | split partials];
//  * persistent: the 256 x 256 persistent kernels (at least half the CUs'
//    worth of tiles, whole stages, N % 4 == 0, 31-bit buffer offsets), f32
//    activations rounded to operand_type() into the workspace first; from
//    kW16MinTokens tokens two-pass (the 16-bit weight image after them in
//    the workspace);
//  * otherwise the tiled kernel, split-K partials in the workspace.
// With a workspace limit (the no-allocation entry point's fixed array) the
// plan keeps within it: the two-pass path only when its image fits, as many
// splits as fit (none if fewer than two), and the tiled kernel (which reads
// f32 activations in place) when the 16-bit copy of f32 activations for the
// persistent kernels does not fit.
struct GemmPlan {
    bool persistent, two_pass, convert_x, skinny, few;
    uint32_t xt;                  // activation type the kernel reads
    TilePlan tiles;               // the tiled kernel's tile and splits (not persistent)
    uint32_t splits;              // the skinny kernel's K splits
    size_t x16_off, img_off, ws;  // workspace: [x16 | image] (persistent), [packed x | partials]
                                  // (skinny), split-K partials (tiled)
};
constexpr size_t kNoWorkspaceLimit = ~(size_t)0;

inline GemmPlan plan_gemm(uint32_t wtype, uint32_t xtype, uint32_t N, uint32_t K, uint32_t M, int num_cus,
                          size_t ws_limit = kNoWorkspaceLimit) {
    GemmPlan p{};
    p.xt = xtype;
    p.tiles = TilePlan{64, 1};
    p.splits = 1;
    const uint64_t rb = row_bytes_of(wtype, K);
    const bool offsets31 = (uint64_t)M * K * 2u < (1ull << 31) && (uint64_t)N * rb < (1ull << 31);
    const uint64_t tiles = (uint64_t)((M + 255) / 256) * ((N + 255) / 256);
    p.persistent = K % kStageK == 0 && N % 4 == 0 && 2 * tiles >= (uint64_t)num_cus && offsets31;
    if (!p.persistent && few_fits(N, K, M, num_cus) && (uint64_t)(N + kFewFeatures) * rb < (1ull << 32)) {
        p.few = true;
        return p;
    }
    if (!p.persistent && M <= 256 && K % kStageK == 0 && N % 4 == 0 && offsets31) {
        // few tokens over few features: the skinny kernel (one workgroup per
        // CU: its LDS), K split so the launch fills the CUs in one round (at
        // least kSplitMinStages stages per split), as far as the partials fit
        // the workspace
        const size_t x16 = skinny_x_bytes(xtype, M, K), part = (size_t)M * N * sizeof(float);
        if (x16 <= ws_limit) {
            const uint32_t S = K / kStageK, tn = (N + 63) / 64;
            uint32_t want = std::max<uint32_t>(1u, std::min<uint32_t>((uint32_t)num_cus / tn, S / kSplitMinStages));
            if (want > 1 && x16 + want * part > ws_limit)
                want = std::max<uint32_t>(1u, (uint32_t)((ws_limit - x16) / part));
            p.skinny = true;
            p.xt = operand_type(wtype, xtype);
            p.splits = nonempty_splits(S, want);
            p.ws = x16 + (p.splits > 1 ? p.splits * part : 0u);
            return p;
        }
    }
    if (p.persistent && xtype == kF32 && align256((size_t)M * K * 2u) > ws_limit) p.persistent = false;
    if (!p.persistent) {
        p.tiles = plan_tiles(wtype, N, K, M, num_cus);
        const size_t part = (size_t)M * N * sizeof(float);
        if (p.tiles.splits > 1 && (size_t)p.tiles.splits * part > ws_limit) {
            const size_t fit = ws_limit / part;
            p.tiles.splits = fit >= 2 ? nonempty_splits(K / kStageK, (uint32_t)std::min<size_t>(fit, p.tiles.splits))
                                      : 1u;
        }
        p.ws = p.tiles.splits > 1 ? (size_t)p.tiles.splits * part : 0u;
        return p;
    }
    p.convert_x = xtype == kF32;
    p.xt = operand_type(wtype, xtype);
    p.x16_off = 0;
    p.img_off = p.convert_x ? align256((size_t)M * K * 2u) : 0u;
    p.two_pass = M >= kW16MinTokens && p.img_off + w16_image_bytes(N, K, false) <= ws_limit;
    p.ws = p.img_off + (p.two_pass ? w16_image_bytes(N, K, false) : 0u);
    return p;
}

}  // namespace plan
}  // namespace llmr
