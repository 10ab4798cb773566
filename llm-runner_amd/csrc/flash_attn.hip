// flash_attn.hip - non-causal flash attention (head_dim 128) on gfx950 matrix cores.
//
//   O[s, h*128 + d] = sum_j softmax_j(scale * <Q[h,s,:], K[h,j,:]>) V[h,j,d]
//
// Semantics of flash_attention_v2 (dependencies/zimage.c3l/shaders/flash_attn.slang:38-241):
// Q/K/V [H,S,128] rounded to fp16 for the products (the reference rounds
// them to fp16 in its LDS tiles), f32 scores and online softmax state,
// output divided by the row sum, written as f32 [S, H*128] (reverse head
// transpose fused). One kernel, flash_attn_fwd64_w8, on fp16 K/V; f32 and
// bf16 K and V are rounded to fp16 (nearest even) by one conversion pass into
// the context workspace first, and f32 / bf16 Q as the kernel loads it
// (once per workgroup): the reference rounds Q/K/V to fp16 in its LDS
// tiles, so the result is the same.
#include <type_traits>

#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

constexpr int kD = 128;


// ---------------------------------------------------------------------------
// fp16 fast path: 256 queries per workgroup, DMA-fed LDS rings.
//
// A workgroup of 8 / NB waves takes 256 queries of one head; each wave owns
// NB blocks of 32 queries (NB = 1: 8 waves, two per SIMD; the kernel is
// written for any NB, and with NB = 2 every K or V fragment read from LDS
// feeds two MFMAs). K and V tiles of 64 keys go HBM -> LDS by buffer DMA
// (no staging registers, no VALU) into 3-slot rings, K three tiles and V two
// tiles ahead of use; V stays row-major in LDS and the V^T operand is read
// with the transposing ds_read_b64_tr_b16 (lane i of a 16-lane group gets
// V[key0 + e][d0 + i], e = 0..3).
//
// Scores live in three 32-key halves used in rotation, so the MFMAs of
// S(t+1) = K(t+1) Q^T go to a free half while S(t) is exponentiated. Per
// tile t a wave: DMAs K(t+3) and V(t+2); computes S(t+1) on the matrix
// cores while the vector ALU exponentiates S(t) into the fp16 P(t);
// accumulates O^T += V(t)^T P(t)^T while taking the row max of S(t+1);
// rescales O if a running max grew by more than 2^8 (lazily: O and the row
// sum keep a stale max until then, exp2 of at most 2^8 cannot overflow);
// then one barrier. The main loop is unrolled by 3 (the
// halves) and walks the LDS rings with scalar slot offsets. It runs while
// S(t+1) has no keys past the sequence end; one masked iteration follows
// when the last tile is partial, then a final iteration that only
// exponentiates and accumulates.
// ---------------------------------------------------------------------------
constexpr uint32_t kBQ64 = 256;            // queries per workgroup
constexpr uint32_t kTile64 = 64u * 256u;   // one K or V tile: 64 keys x 128 fp16
// LDS of a workgroup: the K and V rings (6 tiles), or the epilogue's
// staging of the output rows (kBQ64 queries x 128 f32)
constexpr uint32_t kFaLds = kBQ64 * 128u * 4u > 6u * kTile64 ? kBQ64 * 128u * 4u : 6u * kTile64;

// LDS rows are 256 bytes (16 chunks of 8 fp16). K: chunk c of key r at
// c ^ (r & 15) (a 16-lane fragment read touches 16 distinct bank quads).
// V: chunk c of key r at c ^ vswz(r); a transposing read touches 8
// consecutive keys x 4 chunks, and vswz spreads those 32 cells evenly over
// the 16 chunk positions (two each: the minimum for 512 bytes).
__device__ __forceinline__ uint32_t kswz(uint32_t r) { return r & 15u; }
__device__ __forceinline__ uint32_t vswz(uint32_t r) { return ((r & 3u) << 2) | ((r >> 2) & 1u); }

__device__ __forceinline__ float xhalf_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));


// QT: type of Q (F16, or F32 / BF16 rounded to fp16 as the fragments are
// loaded: Q is read once per workgroup, so it needs no conversion pass)
// OT: type of the output rows (F32, or F16 / BF16 rounded to nearest even)
// at row stride ostride elements, head h at columns h * 128 of a row
template <int NB, uint32_t QT, uint32_t OT = kGgmlF32>  // query blocks of 32 per wave; 8 / NB waves per workgroup
__device__ __forceinline__ void fa64_body(const void* __restrict__ Q, const _Float16* __restrict__ K,
                                          const _Float16* __restrict__ V, void* __restrict__ O, uint32_t ostride,
                                          uint32_t S,
                                          uint32_t H, float scale_log2, uint32_t n_qb) {
    // K ring in slots 0..2, V ring in slots 3..5
    // (after the key loop the epilogue stages O in it: 16 KiB per 32 queries)
    __shared__ __attribute__((aligned(16))) uint8_t lds[kFaLds];
    constexpr uint32_t ROW = kD * 2u;  // bytes per token row of one head

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t l32 = lane & 31u, kh = lane >> 5;

    // workgroup -> (head, query block), all blocks of a head on one XCD
    const uint32_t total = n_qb * H;
    uint32_t L = blockIdx.x;
    if (total % 8u == 0) L = (L % 8u) * (total / 8u) + L / 8u;
    const uint32_t head = L / n_qb, qb = L % n_qb;
    const uint64_t head_bytes = (uint64_t)S * ROW;
    constexpr uint32_t QB = QT == kGgmlF32 ? 4u : 2u;  // bytes per Q element
    const uint8_t* Qh = (const uint8_t*)Q + head * (uint64_t)S * kD * QB;
    const uint8_t* Kh = (const uint8_t*)K + head * head_bytes;
    const uint8_t* Vh = (const uint8_t*)V + head * head_bytes;
    constexpr uint32_t DI = 2u * NB;      // DMA instructions per tile per wave (64 / W keys)
    const uint32_t q0 = qb * kBQ64 + wave * 32u * NB;  // first query of this wave

    // Q fragments (B operand of S^T = K Q^T) of the two query blocks:
    // d = 32c + 16kh + 8st + 0..7 of query q0 + 32b + l32
    f16x8 qf[NB][4][2];
    {
        const rsrc_t qr = make_rsrc(Qh, (uint64_t)S * kD * QB);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    const uint32_t off = ((q0 + 32u * b + l32) * kD + 32u * c + 16u * kh + 8u * st) * QB;
                    f32x4 a, e;  // the 8 elements as f32 (exact for f16 / bf16 inputs)
                    if constexpr (QT == kGgmlF32) {
                        a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0));
                        e = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off + 16u, 0, 0));
                    } else {
                        const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, 0));
                        // the components by name: indexed as w[k] in this
                        // unrolled loop, hipcc read w[0] for every k
                        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
                        float x[8];
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            if constexpr (QT == kGgmlBF16) {
                                x[2 * k] = __uint_as_float(wd[k] << 16);
                                x[2 * k + 1] = __uint_as_float(wd[k] & 0xffff0000u);
                            } else {
                                const f16x2 hw = __builtin_bit_cast(f16x2, wd[k]);
                                x[2 * k] = (float)hw.x;
                                x[2 * k + 1] = (float)hw.y;
                            }
                        }
                        a = f32x4{x[0], x[1], x[2], x[3]};
                        e = f32x4{x[4], x[5], x[6], x[7]};
                    }
                    if constexpr (QT != kGgmlF16) {  // rounded to fp16 first, as the fp16 inputs are
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            a[k] = (float)(_Float16)a[k];
                            e[k] = (float)(_Float16)e[k];
                        }
                    }
                    // the softmax scale (log2 domain) carried by Q: the score
                    // MFMAs then produce exp2's argument
                    a *= scale_log2;
                    e *= scale_log2;
                    qf[b][c][st] = __builtin_bit_cast(f16x8, u32x4{pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w),
                                                                  pack_f16x2(e.x, e.y), pack_f16x2(e.z, e.w)});
                }
    }

    // DMA lane offsets: instruction i of wave w fills keys 4(DI w + i) +
    // lane/16 of a slot, lane l landing in physical chunk l % 16 of its key
    uint32_t kvo[DI], vvo[DI];
#pragma unroll
    for (int i = 0; i < (int)DI; i++) {
        const uint32_t r = 4u * (DI * wave + i) + (lane >> 4), p = lane & 15u;
        kvo[i] = r * ROW + ((p ^ kswz(r)) << 4);
        vvo[i] = r * ROW + ((p ^ vswz(r)) << 4);
    }
    // tile t's keys through a descriptor ending at the sequence end (keys
    // past it, and tiles past the last, read as zero) into LDS slot `slot`
    auto dma = [&](const uint8_t* base, const uint32_t (&vo)[DI], uint32_t t, uint32_t slot) {
        const uint32_t k0 = t * 64u;
        // S * ROW < 2^32 (checked by the host); readfirstlane keeps the
        // descriptor in scalar registers
        const uint32_t bytes = __builtin_amdgcn_readfirstlane(k0 < S ? (S - k0) * ROW : 0u);
        const rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base) + (uint64_t)k0 * ROW,
                                                           (short)0, (int)bytes, 0x00020000);
        uint8_t* dst = lds + slot * kTile64 + wave * (4u * DI * ROW);
#pragma unroll
        for (int i = 0; i < (int)DI; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(dst + 1024u * i), 16, vo[i], 0, 0, 0);
    };

    // K fragment offsets (A operand of S^T): key 32kb + l32 (+ 32kb*ROW at use),
    // chunk 4c + 2kh + st
    uint32_t kfo[4][2];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int st = 0; st < 2; st++) kfo[c][st] = l32 * ROW + (((4u * c + 2u * kh + st) ^ kswz(l32)) << 4);
    // V^T fragment offsets (transposing reads): lane (group g, index j)
    // addresses key R + 4(g/2) + j/4 (R = 32kb + 16c + 8h at use), dims
    // 32dt + 16(g%2) + 4(j%4) .. +3
    uint32_t vto[4];
    {
        const uint32_t g = lane >> 4, j = lane & 15u;
        const uint32_t kr = 4u * (g >> 1) + (j >> 2);
        const uint32_t x = 2u * (g & 1u) + ((j & 3u) >> 1), half = j & 1u;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) vto[dt] = kr * ROW + (((4u * dt + x) ^ vswz(kr)) << 4) + 8u * half;
    }

    // Scores are kept relative to m_ref, the max the exponentials use (log2
    // domain; Q carries the scale): the score MFMAs start from -m_ref
    // instead of zero, so a score is exp2's argument as it stands.
    f32x16 o[4][NB];
    float m_ref[NB], l_i[NB];  // this lane's query's m_ref; its partial row sums
#pragma unroll
    for (int b = 0; b < NB; b++) {
        m_ref[b] = 0.0f;
        l_i[b] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt][b] = f32x16{};
    }

    // Score halves: the scores of one 32-key block of a tile for both query
    // blocks; h[b] at lane l holds key 32kb + 8(i/4) + 4kh + i%4 of the
    // tile (kb = the block), query 32b + l32.
    //
    // K fragment f = 0..15 of the tile at Ks: key block f/8, d chunk
    // (c, st) = ((f%8)/2, f%2)
    auto kfrag = [&](const uint8_t* Ks, int f) -> f16x8 {
        return *(const f16x8*)(Ks + 32u * (uint32_t)(f / 8) * ROW + kfo[(f % 8) / 2][f % 2]);
    };
    // V^T fragment f = 0..15 of the tile at Vs: key block kb = f/8, keys
    // 32kb + 16c + {4kh..4kh+3, 8+4kh..8+4kh+3} with c = (f%8)/4, dims
    // 32dt + l32 with dt = f%4
    auto vfrag = [&](const uint8_t* Vs, int f) -> f16x8 {
        const uint32_t R = 32u * (uint32_t)(f / 8) + 16u * (uint32_t)((f % 8) / 4);
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(Vs + R * ROW + vto[f % 4]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(Vs + (R + 8u) * ROW + vto[f % 4]));
        return __builtin_bit_cast(
            f16x8, (short __attribute__((ext_vector_type(8)))){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w});
    };
    // S of the tile at Ks into the halves (h0: keys 0..31, h1: keys 32..63)
    auto qk_all = [&](const uint8_t* Ks, f32x16 (&h0)[NB], f32x16 (&h1)[NB]) {
        static_for<0, 16>([&](auto F) {
            constexpr int f = F, kb = f / 8, c = (f % 8) / 2, st = f % 2;
            const f16x8 a = kfrag(Ks, f);
            static_for<0, NB>([&](auto B) {
                constexpr int b = B;
                f32x16& s = kb == 0 ? h0[b] : h1[b];
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[b][c][st], (c == 0 && st == 0) ? f32x16{} : s,
                                                           0, 0, 0);
            });
        });
    };
    // keys >= S of tile t (halves h0, h1) to -inf
    auto mask = [&](f32x16 (&h0)[NB], f32x16 (&h1)[NB], uint32_t t) {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t key = t * 64u + 8u * (i >> 2) + 4u * kh + (i & 3);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                h0[b][i] = key < S ? h0[b][i] : -INFINITY;
                h1[b][i] = key + 32u < S ? h1[b][i] : -INFINITY;
            }
        }
    };
    // row max of a tile's scores (relative to m_ref), both halves of the wave
    // combined
    auto rowmax = [&](const f32x16 (&h0)[NB], const f32x16 (&h1)[NB], float (&mx)[NB]) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float m = h0[b][0];
#pragma unroll
            for (int i = 0; i < 16; i++) m = fmaxf(fmaxf(m, h0[b][i]), h1[b][i]);
            mx[b] = xhalf_max(m);
        }
    };
    // raise m_ref where the tile whose scores are in (n0, n1) exceeds it by
    // more than 2^8 (lazily: exp2 of at most 2^8 cannot overflow), and shift
    // those scores to the new m_ref (the next tile's MFMAs start from it)
    auto rescale = [&](const float (&mx)[NB], f32x16 (&n0)[NB], f32x16 (&n1)[NB]) {
        bool grow = false;
#pragma unroll
        for (int b = 0; b < NB; b++) grow = grow || mx[b] > 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float d = fmaxf(mx[b], 0.0f);
                const float alpha = __builtin_amdgcn_exp2f(-d);
                m_ref[b] += d;
                l_i[b] *= alpha;
#pragma unroll
                for (int dt = 0; dt < 4; dt++) o[dt][b] *= alpha;
                n0[b] -= d;
                n1[b] -= d;
            }
        }
    };
    // P = exp2(score) of score pair `item` (query block item/8, keys
    // 2(item%8), +1) of half h (key block kb) into the fp16 operand p
    // (p[b][kb][c] holds keys 16c..16c+15 of the block); row sums into rs
    // (as one v_dot2 of the fp16 pair with (1, 1) instead of the two adds:
    // 0.2595-0.2621 against 0.2556-0.2562 ms, three alternating runs each
    // on one box)
    auto exp_pair = [&](const f32x16 (&h)[NB], int kb, int item, f16x8 (&p)[NB][2][2], float (&rs)[NB]) {
        const int b = item / 8, i = 2 * (item % 8);
        const float e0 = __builtin_amdgcn_exp2f(h[b][i]);
        const float e1 = __builtin_amdgcn_exp2f(h[b][i + 1]);
        const f16x2 pe{(_Float16)e0, (_Float16)e1};
        rs[b] += e0 + e1;
        p[b][kb][i >> 3][i & 7] = pe.x;
        p[b][kb][i >> 3][(i & 7) + 1] = pe.y;
    };

    // One tile t. S(t) is in (c0, c1); S(t+1) = K(t+1) Q^T goes to (n0, c0)
    // (n0 free; c0's block-0 scores are exponentiated before its first
    // write). K(t+1) is in LDS slot ks, V(t) in V slot vs; K(t+3) is DMAed
    // to K slot kd and V(t+2) to V slot vd.
    // The 32 NB MFMAs (16 NB for S(t+1), then 16 NB for O^T += V(t)^T P(t)^T)
    // are issued in a fixed order with the vector work spread between them:
    // the exponentials of block 0 under the first 8 NB, those of block 1
    // under the next 16 NB (P's block 0 is complete before its accumulation
    // starts), then the row max of S(t+1) under the accumulation MFMAs.
    // Fragment reads run PF fragments ahead of their MFMAs. sched_barrier
    // fences keep that order.
    auto tile = [&](f32x16 (&c0)[NB], f32x16 (&c1)[NB], f32x16 (&n0)[NB], uint32_t t, uint32_t ks, uint32_t vs,
                    uint32_t kd, uint32_t vd, auto masked) {
        dma(Kh, kvo, t + 3u, kd);
        dma(Vh, vvo, t + 2u, 3u + vd);
        const uint8_t* Ks = lds + ks * kTile64;
        const uint8_t* Vs = lds + (3u + vs) * kTile64;
        f16x8 p[NB][2][2];
        constexpr int PF = 3;  // fragments in flight ahead of their MFMAs
        constexpr int QS = 16 * NB;  // steps of the score MFMAs (then as many accumulation steps)
        f16x8 kf[PF + 1], vf[PF + 1];
        float rs[NB], mt[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            rs[b] = 0.0f;
            mt[b] = -INFINITY;
        }
        static_for<0, PF>([&](auto F) { kf[F] = kfrag(Ks, F); });
        static_for<0, 2 * QS>([&](auto J) {
            constexpr int j = J;
            if constexpr (j < QS) {
                constexpr int f = j / NB, b = j % NB, kb = f / 8, c = (f % 8) / 2, st = f % 2;
                if constexpr (b == 0 && f + PF < 16) kf[(f + PF) % (PF + 1)] = kfrag(Ks, f + PF);
                f32x16& s = kb == 0 ? n0[b] : c0[b];
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[f % (PF + 1)], qf[b][c][st],
                                                           (c == 0 && st == 0) ? f32x16{} - m_ref[b] : s, 0, 0,
                                                           0);
            } else {
                constexpr int f = (j - QS) / NB, b = j % NB, kb = f / 8, c = (f % 8) / 4, dt = f % 4;
                if constexpr (b == 0 && f + PF < 16) vf[(f + PF) % (PF + 1)] = vfrag(Vs, f + PF);
                o[dt][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[f % (PF + 1)], p[b][kb][c], o[dt][b], 0, 0, 0);
            }
            if constexpr (j >= QS - PF && j < QS) vf[j - (QS - PF)] = vfrag(Vs, j - (QS - PF));
            if constexpr (j < 8 * NB) exp_pair(c0, 0, j, p, rs);
            if constexpr (j >= 8 * NB && j < 24 * NB && j % 2 == 0) exp_pair(c1, 1, (j - 8 * NB) / 2, p, rs);
            if constexpr (decltype(masked)::value && j == QS - 1) mask(n0, c0, t + 1u);
            if constexpr (j >= QS && j % 2 == 0) {
                // row max item k: half k/(4NB) (n0, then c0), query block (k%(4NB))/4, scores 4(k%4)..+3
                constexpr int k = (j - QS) / 2, b = (k % (4 * NB)) / 4, i = 4 * (k % 4);
                const f32x16& s = k < 4 * NB ? n0[b] : c0[b];
                mt[b] = fmaxf(fmaxf(mt[b], s[i]), s[i + 1]);
                mt[b] = fmaxf(fmaxf(mt[b], s[i + 2]), s[i + 3]);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        float mx[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            l_i[b] += rs[b];
            mx[b] = xhalf_max(mt[b]);
        }
        rescale(mx, n0, c0);
        LLMR_STAGE_BARRIER(4 * NB);
    };

    const uint32_t n_tiles = (S + 63u) / 64u;
    const bool partial = (S % 64u) != 0u;
    // iterations t whose S(t+1) has no key past the sequence end
    const uint32_t n_plain = partial ? (n_tiles >= 2u ? n_tiles - 2u : 0u) : n_tiles - 1u;

    // prologue: K(0) V(0) K(1) V(1) K(2) in flight; S(0) and its max
    dma(Kh, kvo, 0, 0);
    dma(Vh, vvo, 0, 3);
    dma(Kh, kvo, 1, 1);
    dma(Vh, vvo, 1, 4);
    dma(Kh, kvo, 2, 2);
    LLMR_STAGE_BARRIER(8 * NB);  // K(0) has landed
    f32x16 h0[NB], h1[NB], h2[NB];
    {   // S(0) from zero; its row max becomes m_ref, S(0) relative to it
        float mx[NB];
        qk_all(lds, h0, h1);
        if (n_tiles == 1u && partial) mask(h0, h1, 0);
        rowmax(h0, h1, mx);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            m_ref[b] = mx[b];
            h0[b] -= mx[b];
            h1[b] -= mx[b];
        }
    }
    LLMR_STAGE_BARRIER(4 * NB);  // K(1), V(0) have landed; every wave is done with K(0)

    // t % 3 = r0 names the ring slots: K(t+1) in r1, V(t) in r0; K(t+3) to
    // r0 (K(t), last read in iteration t-1), V(t+2) to r2 (V(t-1)). The
    // score halves rotate with period 3: S(t) in (h0, h1), (h2, h0), (h1, h2).
    uint32_t t = 0, r0 = 0;
    auto step = [&](f32x16 (&c0)[NB], f32x16 (&c1)[NB], f32x16 (&n0)[NB], auto masked) {
        const uint32_t r1 = r0 == 2u ? 0u : r0 + 1u;
        const uint32_t r2 = r0 == 0u ? 2u : r0 - 1u;
        tile(c0, c1, n0, t, r1, r0, r0, r2, masked);
        t++;
        r0 = r1;
    };
    // S(t) back into (h0, h1) after one step from (h0, h1)
    auto rotate = [&]() {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            h1[b] = h0[b];
            h0[b] = h2[b];
        }
    };
    while (t + 3u <= n_plain) {
        step(h0, h1, h2, std::false_type{});
        step(h2, h0, h1, std::false_type{});
        step(h1, h2, h0, std::false_type{});
    }
    while (t < n_plain) {
        step(h0, h1, h2, std::false_type{});
        rotate();
    }
    if (partial && n_tiles >= 2u) {
        step(h0, h1, h2, std::true_type{});
        rotate();
    }
    {   // last tile: S(n-1) is in (h0, h1), V(n-1) in V slot r0
        f16x8 p[NB][2][2];
        float rs[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) rs[b] = 0.0f;
        static_for<0, 8 * NB>([&](auto I) { exp_pair(h0, 0, I, p, rs); });
        static_for<0, 8 * NB>([&](auto I) { exp_pair(h1, 1, I, p, rs); });
#pragma unroll
        for (int b = 0; b < NB; b++) l_i[b] += rs[b];
        const uint8_t* Vs = lds + (3u + r0) * kTile64;
        static_for<0, 16>([&](auto F) {
            constexpr int f = F, kb = f / 8, c = (f % 8) / 4, dt = f % 4;
            const f16x8 a = vfrag(Vs, f);
            static_for<0, NB>([&](auto B) {
                o[dt][B] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, p[B][kb][c], o[dt][B], 0, 0, 0);
            });
        });
    }
    LLMR_WAIT_VMCNT(0);  // no DMA may still be writing LDS when the wave exits

    // O = O^T / l through LDS: the lanes hold 16-byte pieces of 32 query
    // rows (query l32, dims 32 dt + 8 g + 4 kh + 0..3); stored as they are,
    // every store instruction would write 32-byte pieces of 32 rows 12 KiB
    // apart. Each wave stages its rows in its own 16 KiB per query block
    // (row r at r * 512 bytes, 16-byte chunk c at (c ^ (r % 32)) * 16) once
    // every wave is done with the K/V rings, and stores two whole 512-byte
    // rows per instruction (flux_attention 0.315 -> 0.309 ms, mean of three
    // runs each on one box).
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float* const ot = (float*)lds + (wave * NB + b) * (32u * kD);
        const float inv_l = 1.0f / xhalf_sum(l_i[b]);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t c = 8u * dt + 2u * g + kh;
                *(f32x4*)(ot + l32 * kD + ((c ^ l32) << 2)) =
                    f32x4{o[dt][b][4 * g] * inv_l, o[dt][b][4 * g + 1] * inv_l, o[dt][b][4 * g + 2] * inv_l,
                          o[dt][b][4 * g + 3] * inv_l};
            }
    }
    // the wave reads back only what it wrote: its LDS operations run in order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const float* const ot = (const float*)lds + (wave * NB + b) * (32u * kD);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t r = 2u * i + kh, q = q0 + 32u * b + r;
            const f32x4 v = *(const f32x4*)(ot + r * kD + ((l32 ^ r) << 2));
            if (q >= S) continue;
            const uint64_t at = (uint64_t)q * ostride + (uint64_t)head * kD + 4u * l32;
            if constexpr (OT == kGgmlF32) {
                *(f32x4*)((float*)O + at) = v;
            } else if constexpr (OT == kGgmlBF16) {
                typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
                *(u32x2*)((uint16_t*)O + at) = u32x2{__builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)v.x, (__bf16)v.y}),
                                                     __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)v.z, (__bf16)v.w})};
            } else {
                *(u32x2*)((uint16_t*)O + at) = u32x2{pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w)};
            }
        }
    }
}
// 8 waves of 32 queries: two waves per SIMD, so one wave's softmax runs
// beside the other's MFMAs (measured 827 vs 737 TFLOP/s for 4 waves of 64
// queries at H = 24, S = 4608, which also need 495 of the 512 registers)
template <uint32_t QT, uint32_t OT = kGgmlF32>
__global__ void __launch_bounds__(512, 1)
flash_attn_fwd64_w8(const void* __restrict__ Q, const _Float16* __restrict__ K, const _Float16* __restrict__ V,
                    void* __restrict__ O, uint32_t ostride, uint32_t S, uint32_t H, float scale_log2,
                    uint32_t n_qb) {
    fa64_body<1, QT, OT>(Q, K, V, O, ostride, S, H, scale_log2, n_qb);
}

// K and V (blockIdx.y = 0, 1) of f32 or bf16 type -> fp16, round to nearest
// even; 8 elements per thread.
template <uint32_t XT>
__global__ void __launch_bounds__(256) kv_to_f16_kernel(const void* __restrict__ k, const void* __restrict__ v,
                                                        u32x4* __restrict__ out, size_t n8) {
    const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= n8) return;
    const void* src = blockIdx.y == 0 ? k : v;
    u32x4 r;
    if constexpr (XT == kGgmlF32) {
        const f32x4 a = ((const f32x4*)src)[2 * i], b = ((const f32x4*)src)[2 * i + 1];
        r = u32x4{pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y), pack_f16x2(b.z, b.w)};
    } else {
        const u32x4 w = ((const u32x4*)src)[i];
        r = u32x4{bf16x2_to_f16x2(w.x), bf16x2_to_f16x2(w.y), bf16x2_to_f16x2(w.z), bf16x2_to_f16x2(w.w)};
    }
    out[(size_t)blockIdx.y * n8 + i] = r;
}

}  // namespace

size_t flash_attention_workspace_bytes(uint32_t xtype, uint32_t n_heads, uint32_t seq_len) {
    return xtype == kGgmlF16 ? 0u : 2u * (size_t)n_heads * seq_len * kD * 2u;
}

hipError_t launch_flash_attention(const void* q, const void* k, const void* v, uint32_t xtype,
                                  void* o, uint32_t otype, uint32_t ostride, uint32_t n_heads, uint32_t seq_len,
                                  float scale, void* ws, hipStream_t st) {
    if (seq_len == 0 || n_heads == 0) return hipSuccess;
    if (xtype != kGgmlF16) {  // K and V to fp16 in the workspace; Q is converted as it is loaded
        const size_t n8 = (size_t)n_heads * seq_len * kD / 8u;
        const dim3 grid((uint32_t)((n8 + 255) / 256), 2);
        if (xtype == kGgmlF32)
            hipLaunchKernelGGL(kv_to_f16_kernel<kGgmlF32>, grid, dim3(256), 0, st, k, v, (u32x4*)ws, n8);
        else
            hipLaunchKernelGGL(kv_to_f16_kernel<kGgmlBF16>, grid, dim3(256), 0, st, k, v, (u32x4*)ws, n8);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        k = ws;
        v = (const u32x4*)ws + n8;
    }
    const float scale_log2 = scale * 1.4426950408889634f;
    const uint32_t n_qb64 = (seq_len + kBQ64 - 1) / kBQ64;
    const dim3 grid(n_qb64 * n_heads), block(512);
    const _Float16 *kh = (const _Float16*)k, *vh = (const _Float16*)v;
    auto go = [&](auto qt, auto ot) {
        hipLaunchKernelGGL((flash_attn_fwd64_w8<decltype(qt)::value, decltype(ot)::value>), grid, block, 0, st, q, kh,
                           vh, o, ostride, seq_len, n_heads, scale_log2, n_qb64);
    };
    using F32 = std::integral_constant<uint32_t, kGgmlF32>;
    using F16 = std::integral_constant<uint32_t, kGgmlF16>;
    using BF16 = std::integral_constant<uint32_t, kGgmlBF16>;
    auto by_out = [&](auto qt) {
        if (otype == kGgmlBF16) go(qt, BF16{});
        else if (otype == kGgmlF16) go(qt, F16{});
        else go(qt, F32{});
    };
    if (xtype == kGgmlF32) by_out(F32{});
    else if (xtype == kGgmlBF16) by_out(BF16{});
    else by_out(F16{});
    return hipGetLastError();
}

}  // namespace llmr
