// Dequant-GEMM for few tokens (M <= 256): batch_matmul_q8 / batch_matmul_q4k
// (llm.slang:1639-1767, :2277-2365) when the output has too few 256 x 256
// tiles for the persistent kernels, e.g. a single linear over 256 tokens.
//
// Workgroup (n tile, split z) computes all M tokens x 64 features over the K
// stages [z per, min(S, (z + 1) per)): the activations are read by N / 64
// workgroups (not by N / 64 x M / 64 as with square tiles), and the launch
// splits K until every CU has a workgroup; the partial tiles are summed in
// split order by splitk_reduce_kernel. Eight waves, two per SIMD (one
// wave's copies, dequantization and waits overlap the other's MFMAs): wave
// w holds tokens 32 w .. 32 w + 31 x the 64 features in two 32x32x16 MFMA
// accumulators.
//  * 16-bit activations are read where they are (row-major); f32 ones are
//    first rounded to the operand type (fp16 against Q8_0: the reference's
//    float16_t(v); bf16 against Q4_K, whose reference keeps x in f32) into
//    the workspace, stage-major, [K / 64][M][64]: a stage's slab is one
//    contiguous M x 128-byte block;
//  * everything goes HBM -> LDS by buffer_load ... lds (no loads into
//    registers in the stage loop, so the compiler adds no waits of its own):
//    activations into a 4-slot ring, wave w copying its own 32 token rows
//    (the rows it multiplies) with each lane's source offset permuted so
//    the fixed lane * 16 LDS placement realizes the bank swizzle; the packed
//    weight bytes of the tile's 64 rows into a 3-slot ring, as [row][RD
//    dwords], copied by waves 0-5;
//  * a stage's packed weights are dequantized one stage ahead by waves 0-3
//    (thread (wave w, lane l): part w of row l, LDS chunks w and 4 + w,
//    with the fused kernels' WRow code) into a 2-slot ring of 16-bit
//    operands;
//  * stage g issues stage g+3's copies; its one barrier waits until only
//    those are in flight.
// Rows past M and features past N read as zero through the buffer
// descriptors and are not stored.
#include "gemm_q_common.h"
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

constexpr uint32_t kSkX = 256u * 128u;  // one activation stage: 256 rows x 64 k x 2 bytes
constexpr uint32_t kSkW = 64u * 128u;   // one 16-bit weight stage: 64 rows x 64 k x 2 bytes
constexpr uint32_t kSkXSlots = 4, kSkRSlots = 3, kSkWSlots = 2;

// Packed weight bytes of one row and stage: RD dwords, copied by RI DMAs
// of 64 dwords in each of waves 0-5 (6 RI >= RD; the spare lanes copy
// zeros).
//   Q8_0: blocks 2s, 2s+1 = 68 bytes at 68 s (WRow<Q8_0>'s a, b, c, d, e);
//   Q4_K: superblock s/4's 16-byte header, then its 32 quant bytes at
//         16 + 32 (s % 4) (WRow<Q4_K>'s hdr, qa, qb).
template <uint32_t WT>
struct SkRaw {
    static constexpr uint32_t kWaves = 6;  // the waves that copy
    static constexpr uint32_t RD = WT == kGgmlQ8_0 ? 17u : 12u, RI = (RD + kWaves - 1) / kWaves;
    static constexpr uint32_t kSlot = kWaves * RI * 256u;  // bytes of one ring slot
    // byte offset of dword dw of a row (before the row's own offset) and
    // the uniform stage offset
    __device__ static uint32_t voff(uint32_t dw, uint32_t s) {
        if constexpr (WT == kGgmlQ8_0) return 4u * dw;
        else return dw < 4u ? 4u * dw : 16u + 32u * (s & 3u) + 4u * (dw - 4u);
    }
    __device__ static uint32_t soff(uint32_t s) { return WT == kGgmlQ8_0 ? 68u * s : (s >> 2) * 144u; }
    template <uint32_t OT>
    __device__ static WRow<WT, OT> row(const uint8_t* slot, uint32_t r) {
        const uint32_t* const q = (const uint32_t*)(slot + r * RD * 4u);
        WRow<WT, OT> w;
        if constexpr (WT == kGgmlQ8_0) {
            w.a = u32x4{q[0], q[1], q[2], q[3]};
            w.b = u32x4{q[4], q[5], q[6], q[7]};
            w.c = u32x4{q[8], q[9], q[10], q[11]};
            w.d = u32x4{q[12], q[13], q[14], q[15]};
            w.e = q[16];
        } else {
            w.hdr = u32x4{q[0], q[1], q[2], q[3]};
            w.qa = u32x4{q[4], q[5], q[6], q[7]};
            w.qb = u32x4{q[8], q[9], q[10], q[11]};
        }
        return w;
    }
};

template <uint32_t WT, uint32_t XT>
__global__ void __launch_bounds__(512, 1)
    gemm_q_skinny(const uint8_t* __restrict__ W, const void* __restrict__ X, float* __restrict__ Y, uint32_t N,
                  uint32_t K, uint32_t M, uint32_t row_offset, uint32_t per, uint64_t split_stride,
                  bool stage_major) {
    static_assert(XT == kGgmlF16 || XT == kGgmlBF16, "16-bit activations only");
    using R = SkRaw<WT>;
    constexpr uint32_t RI = R::RI;
    // one LDS object (a second one makes the compiler wait for every DMA)
    __shared__ __attribute__((aligned(16)))
    uint8_t lds[kSkXSlots * kSkX + kSkRSlots * R::kSlot + kSkWSlots * kSkW];
    uint8_t* const Xs = lds;
    uint8_t* const Rs = lds + kSkXSlots * kSkX;
    uint8_t* const Ws = Rs + kSkRSlots * R::kSlot;

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t l32 = lane & 31u, kh = lane >> 5;
    const bool copies_w = wave < R::kWaves, dequantizes = wave < 4u;
    const uint32_t n0 = blockIdx.x * 64u;
    const uint32_t S = K / kBK, s_begin = blockIdx.y * per, s_end = min(S, s_begin + per);
    const uint32_t ns = s_end - s_begin;  // >= 1 (host: splits = ceil(S / per))
    Y += blockIdx.y * split_stride;

    // activation DMA i of wave w: token row 32 w + 8 i + lane / 8 (rows
    // past M: past any range, zeros), physical chunk lane % 8 holding
    // logical chunk (lane % 8) ^ lds_swz(row); a stage is 128 bytes of a
    // row (row-major) or the next M x 128-byte slab (stage-major)
    const uint32_t rstride = stage_major ? 128u : K * 2u, sstride = stage_major ? M * 128u : 128u;
    const rsrc_t xr = make_rsrc(X, (uint64_t)M * K * 2u), x_none = make_rsrc(X, 0);
    uint32_t xvoff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 32u * wave + 8u * i + (lane >> 3);
        xvoff[i] = row < M ? row * rstride + (((lane & 7u) ^ lds_swz(row)) << 4) : 0x80000000u;
    }
    // packed-weight DMA j of wave w < 6: dwords u = 64 (RI w + j) + lane of
    // the slot, row u / RD, dword u % RD (u >= 64 RD: a spare lane)
    const uint32_t rb = (WT == kGgmlQ8_0) ? (K / 32u) * 34u : (K / 256u) * 144u;
    const rsrc_t wr = make_rsrc(W + (uint64_t)(row_offset + n0) * rb, (uint64_t)(N - n0) * rb);
    const rsrc_t w_none = make_rsrc(W, 0);
    uint32_t wrow[RI], wdw[RI];
#pragma unroll
    for (uint32_t j = 0; j < RI; j++) {
        const uint32_t u = 64u * (RI * wave + j) + lane;
        wrow[j] = u < 64u * R::RD ? (u / R::RD) * rb : 0x80000000u;  // spare lanes: past any range
        wdw[j] = u % R::RD;
    }
    // the copies of local stage g (none past the split's last stage)
    auto issue = [&](uint32_t g) {
        const bool live = g < ns;
        const uint32_t s = s_begin + g;
        const rsrc_t xrg = live ? xr : x_none, wrg = live ? wr : w_none;
        uint8_t* const xd = Xs + (g % kSkXSlots) * kSkX + wave * (32u * 128u);
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrg, (lds_void*)(xd + 1024u * i), 16, xvoff[i], s * sstride, 0, 0);
        if (!copies_w) return;
        uint8_t* const rd = Rs + (g % kSkRSlots) * R::kSlot + wave * (RI * 256u);
#pragma unroll
        for (uint32_t j = 0; j < RI; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wrg, (lds_void*)(rd + 256u * j), 4, wrow[j] + R::voff(wdw[j], s),
                                                     R::soff(s), 0, 0);
    };
    // dequantize local stage g: packed slot g % 3 -> 16-bit slot g % 2
    const uint32_t wbase = lane * 128u + (lds_swz(lane) << 4);
    auto dequant = [&](uint32_t g) {
        if (!dequantizes) return;
        const WRow<WT, XT> r = R::template row<XT>(Rs + (g % kSkRSlots) * R::kSlot, lane);
        uint8_t* const dst = Ws + (g % kSkWSlots) * kSkW;
        const auto sc = r.scale(s_begin + g);
        switch (wave) {
            case 0: r.template store<0>(dst, sc, wbase); break;
            case 1: r.template store<1>(dst, sc, wbase); break;
            case 2: r.template store<2>(dst, sc, wbase); break;
            default: r.template store<3>(dst, sc, wbase); break;
        }
    };

    f32x16 acc[2] = {f32x16{}, f32x16{}};
    // the copies one stage issues per wave, and the memory-counter wait
    // that leaves only the latest stage's in flight
    auto stage_barrier = [&]() {
        if (copies_w)
            LLMR_STAGE_BARRIER(4 + RI);
        else
            LLMR_STAGE_BARRIER(4);
    };

    // prologue: copies of stages 0 .. 2; stages 0 and 1 landed (stage 2's
    // copies may fly), stage 0 dequantized
    issue(0);
    issue(1);
    issue(2);
    stage_barrier();
    dequant(0);
    LLMR_STAGE_BARRIER(63);  // the dequantized stage 0 (LDS writes); no copy waited for

    for (uint32_t g = 0; g < ns; g++) {
        // stage g: X slot g % 4, 16-bit W slot g % 2. Copies of stage g+3
        // into X slot (g+3) % 4 and packed slot g % 3 (both last read in
        // stage g-1); stage g+1 dequantized into W slot (g+1) % 2 (read in
        // stage g-1).
        issue(g + 3);
        if (g + 1 < ns) dequant(g + 1);
        const uint8_t* const xs = Xs + (g % kSkXSlots) * kSkX;
        const uint8_t* const ws = Ws + (g % kSkWSlots) * kSkW;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // k step t: chunks 4 (t / 2) + (t % 2) (lanes 0-31) and + 2 (32-63)
            const uint32_t ch = 4u * (t >> 1) + 2u * kh + (t & 1);
            const f16x8 xf = *(const f16x8*)(xs + lds_off(32u * wave + l32, ch));
            f16x8 wf[2];
#pragma unroll
            for (int a = 0; a < 2; a++) wf[a] = *(const f16x8*)(ws + lds_off(32u * a + l32, ch));
#pragma unroll
            for (int a = 0; a < 2; a++) acc[a] = mfma16<XT>(wf[a], xf, acc[a]);
        }
        // stage g+2's copies landed (only stage g+3's in flight): the next
        // stage's activations and the packed weights it dequantizes
        stage_barrier();
    }
    // every copy has landed before the workgroup ends
    LLMR_STAGE_BARRIER(0);

    // Output through LDS (the activation ring is free now): the wave's 32
    // tokens x 64 features go in as its accumulators hold them (lane: token
    // l32, features 32 a + 8 g + 4 kh + 0..3) and come out as whole rows, 16
    // lanes x 16 bytes per token row, so a store instruction writes four
    // 256-byte row segments instead of 32-byte pieces of 32 rows.
    constexpr uint32_t kOutLd = 68u;  // floats per LDS row (16-byte pad: distinct banks)
    float* const ot = (float*)lds + wave * 32u * kOutLd;
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            *(f32x4*)(ot + l32 * kOutLd + 32u * a + 8u * g + 4u * kh) =
                f32x4{acc[a][4 * g], acc[a][4 * g + 1], acc[a][4 * g + 2], acc[a][4 * g + 3]};
    // the wave reads back only what it wrote: its LDS operations run in order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool vec_ok = (N % 4u) == 0u;
    const uint32_t c = 4u * (lane & 15u), n = n0 + c;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t r = 4u * i + (lane >> 4), m = 32u * wave + r;
        if (m >= M) continue;
        const f32x4 v = *(const f32x4*)(ot + r * kOutLd + c);
        float* const yp = Y + (uint64_t)m * N + n;
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

// x [M, K] f32 (row-major) -> OT (fp16 or bf16) [K / 64][M][64] (round to
// nearest even); 8 values per thread
template <uint32_t OT>
__global__ void __launch_bounds__(256) skinny_pack_kernel(const float* __restrict__ x, u32x4* __restrict__ out,
                                                          uint32_t M, uint32_t K, uint32_t n8) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n8) return;
    const uint32_t e = 8u * i, m = e / K, k = e % K;
    const f32x4 a = *(const f32x4*)(x + e), b = *(const f32x4*)(x + e + 4);
    auto pk = [](float u, float v) { return OT == kGgmlBF16 ? pack_bf16x2(u, v) : pack_f16x2(u, v); };
    out[((k / 64u) * M + m) * 8u + (k % 64u) / 8u] = u32x4{pk(a.x, a.y), pk(a.z, a.w), pk(b.x, b.y), pk(b.z, b.w)};
}

}  // namespace

hipError_t launch_gemm_skinny(const void* w, uint32_t wtype, const void* x, uint32_t xtype, float* y, uint32_t N,
                              uint32_t K, uint32_t M, uint32_t row_offset, uint32_t splits, void* ws,
                              hipStream_t st) {
    // splits > 1: the reduction takes four floats per thread (N % 4 == 0)
    if (M == 0 || M > 256 || K % kBK || splits == 0 || (splits > 1 && N % 4u)) return hipErrorInvalidValue;
    const uint32_t S = K / kBK;
    if (!plan::splits_nonempty(S, splits)) return hipErrorInvalidValue;  // every split owns a stage
    const uint32_t per = (S + splits - 1) / splits;
    // f32 activations: rounded to the operand type (fp16 against Q8_0, bf16
    // against Q4_K), stage-major, at the start of the workspace; 16-bit ones
    // are read in place
    const bool pack = xtype == kGgmlF32;
    const uint32_t xt = plan::operand_type(wtype, xtype);
    const void* const x16 = pack ? ws : x;
    float* const part = (float*)((uint8_t*)ws + skinny_x_bytes(xtype, M, K));
    if (pack) {
        const uint32_t n8 = M * K / 8u;
        if (xt == kGgmlBF16)
            hipLaunchKernelGGL(skinny_pack_kernel<kGgmlBF16>, dim3((n8 + 255) / 256), dim3(256), 0, st,
                               (const float*)x, (u32x4*)ws, M, K, n8);
        else
            hipLaunchKernelGGL(skinny_pack_kernel<kGgmlF16>, dim3((n8 + 255) / 256), dim3(256), 0, st,
                               (const float*)x, (u32x4*)ws, M, K, n8);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    const uint64_t mn = (uint64_t)M * N;
    float* const out = splits > 1 ? part : y;
    const dim3 grid((N + 63) / 64, splits);
    if (wtype == kGgmlQ8_0) {
        if (xt == kGgmlBF16)
            hipLaunchKernelGGL((gemm_q_skinny<kGgmlQ8_0, kGgmlBF16>), grid, dim3(512), 0, st, (const uint8_t*)w, x16,
                               out, N, K, M, row_offset, per, splits > 1 ? mn : 0ull, pack);
        else
            hipLaunchKernelGGL((gemm_q_skinny<kGgmlQ8_0, kGgmlF16>), grid, dim3(512), 0, st, (const uint8_t*)w, x16,
                               out, N, K, M, row_offset, per, splits > 1 ? mn : 0ull, pack);
    } else {
        if (xt == kGgmlBF16)
            hipLaunchKernelGGL((gemm_q_skinny<kGgmlQ4K, kGgmlBF16>), grid, dim3(512), 0, st, (const uint8_t*)w, x16,
                               out, N, K, M, row_offset, per, splits > 1 ? mn : 0ull, pack);
        else
            hipLaunchKernelGGL((gemm_q_skinny<kGgmlQ4K, kGgmlF16>), grid, dim3(512), 0, st, (const uint8_t*)w, x16,
                               out, N, K, M, row_offset, per, splits > 1 ? mn : 0ull, pack);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_splitk_reduce(part, y, mn, splits, st);
}

}  // namespace llmr
