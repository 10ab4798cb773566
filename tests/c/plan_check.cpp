// plan_check.cpp - sweeps GEMM shapes through the dispatcher's planner
// (llm-runner_amd/csrc/gemm_plan.h, host code only) and checks what every
// launch relies on:
//  * a split launch gives every split at least one K stage (the kernels
//    load their first stage unconditionally);
//  * the workspace a plan asks for stays within the limit it was given;
//  * f32 activations are rounded to fp16 against Q8_0 (the reference's
//    float16_t(x), llm.slang:1673) and to bf16 against Q4_K (whose reference
//    keeps x in f32, llm.slang:2300-2304).
// Prints "plan_check: N plans ok" and exits 0, or prints the first failing
// case and exits 1.
#include <cstdio>
#include <cstdlib>

#include "gemm_plan.h"

using namespace llmr::plan;

static long n_checked = 0;

static void fail(const char* what, uint32_t wt, uint32_t xt, uint32_t N, uint32_t K, uint32_t M, int cus,
                 size_t limit) {
    std::printf("FAIL %s: wtype %u xtype %u N %u K %u M %u cus %d limit %zu\n", what, wt, xt, N, K, M, cus, limit);
    std::exit(1);
}

static void check(uint32_t wt, uint32_t xt, uint32_t N, uint32_t K, uint32_t M, int cus, size_t limit) {
    const GemmPlan p = plan_gemm(wt, xt, N, K, M, cus, limit);
    const uint32_t S = K / kStageK;
    n_checked++;
    if (p.few + p.skinny + p.persistent > 1) fail("more than one kernel", wt, xt, N, K, M, cus, limit);
    if (p.ws > limit) fail("workspace beyond the limit", wt, xt, N, K, M, cus, limit);
    if (p.few) {
        if (M > kFewMaxTokens || K % kStageK || p.ws != 0) fail("few-token plan", wt, xt, N, K, M, cus, limit);
        return;
    }
    if (p.skinny) {
        if (!splits_nonempty(S, p.splits)) fail("skinny split without stages", wt, xt, N, K, M, cus, limit);
        if (p.splits > 1 && N % 4) fail("skinny split reduction needs N % 4", wt, xt, N, K, M, cus, limit);
        if (xt == kF32 && p.xt != f32_operand_type(wt)) fail("skinny f32 operand type", wt, xt, N, K, M, cus, limit);
        return;
    }
    if (p.persistent) {
        if (xt == kF32 && (!p.convert_x || p.xt != f32_operand_type(wt)))
            fail("persistent f32 operand type", wt, xt, N, K, M, cus, limit);
        if (p.two_pass && M < kW16MinTokens) fail("two-pass below its token count", wt, xt, N, K, M, cus, limit);
        return;
    }
    // the tiled kernel (or, Q8_0 with K % 64 == 32, the generic one: no splits)
    if (wt == kQ8_0 && K % kStageK) {
        if (p.tiles.splits != 1) fail("generic kernel split", wt, xt, N, K, M, cus, limit);
        return;
    }
    if (p.tiles.splits > 1) {
        if (!splits_nonempty(S, p.tiles.splits)) fail("tiled split without stages", wt, xt, N, K, M, cus, limit);
        if (((uint64_t)M * N) % 4) fail("tiled split reduction needs M N % 4", wt, xt, N, K, M, cus, limit);
        if (p.ws != (size_t)p.tiles.splits * M * N * 4) fail("tiled split workspace", wt, xt, N, K, M, cus, limit);
    }
}

int main() {
    // the splitting rule on its own
    for (uint32_t S = 1; S <= 300; S++)
        for (uint32_t want = 1; want <= 80; want++) {
            const uint32_t s = nonempty_splits(S, want);
            n_checked++;
            if (s < 1 || s > want || !splits_nonempty(S, s)) {
                std::printf("FAIL nonempty_splits(%u, %u) = %u\n", S, want, s);
                return 1;
            }
        }
    // the case that had an empty split: M 320, N 640, K 3072 on 256 CUs
    {
        const TilePlan t = plan_tiles(kQ8_0, 640, 3072, 320, 256);
        n_checked++;
        if (!splits_nonempty(3072 / kStageK, t.splits)) {
            std::printf("FAIL plan_tiles(320 x 640 x 3072): %u splits\n", t.splits);
            return 1;
        }
    }
    if (f32_operand_type(kQ8_0) != kF16 || f32_operand_type(kQ4K) != kBF16) {
        std::printf("FAIL f32 operand types\n");
        return 1;
    }
    const uint32_t Ms[] = {1, 2, 4, 5, 17, 31, 32, 33, 64, 100, 200, 255, 256, 257, 320, 500, 512, 1000,
                           1024, 2047, 2048, 3000, 4096, 4352, 4608, 9000};
    const uint32_t Ns[] = {4, 60, 64, 96, 100, 256, 320, 640, 1000, 1536, 3072, 3840, 10240, 11520, 21504};
    const uint32_t Ks[] = {256, 512, 768, 1024, 3072, 3840, 10240, 15360, 32, 96, 3104};
    const int cus[] = {256, 304, 80, 8};
    const size_t limits[] = {kNoWorkspaceLimit, (size_t)32 << 20, (size_t)1 << 20, 0};
    for (uint32_t wt : {kQ8_0, kQ4K})
        for (uint32_t xt : {kF32, kF16, kBF16})
            for (uint32_t M : Ms)
                for (uint32_t N : Ns)
                    for (uint32_t K : Ks) {
                        if (wt == kQ4K && K % 256) continue;
                        if (K % 32) continue;
                        for (int c : cus)
                            for (size_t lim : limits) check(wt, xt, N, K, M, c, lim);
                    }
    std::printf("plan_check: %ld plans ok\n", n_checked);
    return 0;
}
