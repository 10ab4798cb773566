// flash_attn.hip - non-causal flash attention (head_dim 128) on gfx950 matrix cores.
//
//   O[s, h*128 + d] = sum_j softmax_j(scale * <Q[h,s,:], K[h,j,:]>) V[h,j,d]
//
// Semantics of flash_attention_v2 (dependencies/zimage.c3l/shaders/flash_attn.slang:38-241):
// Q/K/V [H,S,128] rounded to fp16 for the products, f32 scores and online
// softmax state, output divided by the row sum, written as f32 [S, H*128]
// (reverse head transpose fused).
//
// Design (one 256-thread workgroup = 4 wave64s per 128 queries of one head):
//  * Each wave owns 32 queries. Scores are computed transposed, S^T = K Q^T,
//    with v_mfma_f32_32x32x16_f16 (K rows as the A operand from LDS, the
//    wave's Q as the B operand held in registers for the whole kernel), so a
//    lane holds one query and 16 of every 32 keys: the row max and row sum
//    are in-lane reductions plus one exchange between the two half-waves.
//  * exp2 with the scale folded into log2(e)*scale; P is rounded to fp16 and
//    used directly as the B operand of O^T += V^T P^T: the accumulator layout
//    of the score MFMA is already the operand layout (no data movement), given
//    that V^T is stored in LDS with the keys of each 16-key chunk permuted
//    (swap of key-index bits 2 and 3) to match it.
//  * K and V tiles of 64 keys are double buffered in LDS (K as [key][d],
//    V transposed to [d][key] while staging), with XOR-swizzled 16-byte
//    chunks; the next tile's global loads are issued before the current
//    tile's matrix work. One barrier per tile.
//  * Workgroups are remapped so all query blocks of a head run on one XCD
//    (its K/V stay in that XCD's L2).
#include "llmr_device.h"
#include "llmr_internal.h"

namespace llmr {

namespace {

constexpr int kD = 128;
constexpr int kBQ = 128;  // queries per workgroup
constexpr int kBKV = 64;  // keys per tile
constexpr uint32_t kKBytes = kBKV * kD * 2;   // K tile [64][128] fp16
constexpr uint32_t kVBytes = kD * kBKV * 2;   // V^T tile [128][64] fp16
constexpr uint32_t kStage = kKBytes + kVBytes;

// K tile: 256-byte rows (16 chunks), swizzle by key & 15.
__device__ __forceinline__ uint32_t k_off(uint32_t key, uint32_t c) {
    return key * 256u + ((c ^ (key & 15u)) << 4);
}
// V^T tile: 128-byte rows (8 chunks), swizzle by d & 7.
__device__ __forceinline__ uint32_t v_off(uint32_t d, uint32_t c) {
    return d * 128u + ((c ^ (d & 7u)) << 4);
}

// 8 consecutive elements of a Q/K/V row as fp16.
template <uint32_t XT>
struct Row8;
template <>
struct Row8<kGgmlF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const void* p, uint64_t e, bool ok) {
        v = ok ? *(const u32x4*)((const uint16_t*)p + e) : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ u32x4 f16() const { return v; }
};
template <>
struct Row8<kGgmlBF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const void* p, uint64_t e, bool ok) {
        v = ok ? *(const u32x4*)((const uint16_t*)p + e) : u32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ u32x4 f16() const {
        return u32x4{bf16x2_to_f16x2(v.x), bf16x2_to_f16x2(v.y), bf16x2_to_f16x2(v.z),
                     bf16x2_to_f16x2(v.w)};
    }
};
template <>
struct Row8<kGgmlF32> {
    f32x4 a, b;
    __device__ __forceinline__ void load(const void* p, uint64_t e, bool ok) {
        const float* f = (const float*)p + e;
        a = ok ? *(const f32x4*)f : f32x4{0, 0, 0, 0};
        b = ok ? *(const f32x4*)(f + 4) : f32x4{0, 0, 0, 0};
    }
    __device__ __forceinline__ u32x4 f16() const {
        return u32x4{pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y),
                     pack_f16x2(b.z, b.w)};
    }
};

// Position of key r (0..15) of a 16-key chunk inside the V^T row: bits 2 and 3
// swapped, so lane half kh finds its 8 keys {4kh..4kh+3, 8+4kh..8+4kh+3} at
// positions 8kh..8kh+7.
__device__ __forceinline__ uint32_t vpos(uint32_t r) {
    return (r & 3u) | (((r >> 3) & 1u) << 2) | (((r >> 2) & 1u) << 3);
}

template <uint32_t XT>
__global__ void __launch_bounds__(256, 2)
flash_attn_fwd(const void* __restrict__ Q, const void* __restrict__ K, const void* __restrict__ V,
               float* __restrict__ O, uint32_t S, uint32_t H, float scale_log2, uint32_t n_qb) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStage];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t l32 = lane & 31u, kh = lane >> 5;

    // workgroup -> (head, query block), all blocks of a head on one XCD
    const uint32_t total = n_qb * H;
    uint32_t L = blockIdx.x;
    if (total % 8u == 0) L = (L % 8u) * (total / 8u) + L / 8u;
    const uint32_t head = L / n_qb, qb = L % n_qb;

    const uint64_t hbase = (uint64_t)head * S * kD;
    const uint32_t q_idx = qb * kBQ + wave * 32u + l32;

    // Q fragments (B operand): d = 32*c + 16*kh + 8*st + 0..7
    f16x8 qf[4][2];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int st = 0; st < 2; st++) {
            Row8<XT> r;
            r.load(Q, hbase + (uint64_t)q_idx * kD + 32 * c + 16 * kh + 8 * st, q_idx < S);
            qf[c][st] = __builtin_bit_cast(f16x8, r.f16());
        }

    // K/V staging: K thread -> (chunk tid&15, keys tid>>4 + 16i); V thread ->
    // (8 dims 8*(tid&15).., 4 keys 4*(tid>>4)..)
    Row8<XT> kr[4], vr[4];
    const uint32_t kc = tid & 15u, krow = tid >> 4;
    const uint32_t vdg = tid & 15u, vkg = tid >> 4;
    auto load_tile = [&](uint32_t t) {
        const uint32_t kv0 = t * kBKV;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t key = kv0 + krow + 16u * i;
            kr[i].load(K, hbase + (uint64_t)key * kD + 8 * kc, key < S);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t key = kv0 + 4u * vkg + i;
            vr[i].load(V, hbase + (uint64_t)key * kD + 8 * vdg, key < S);
        }
    };
    auto store_tile = [&](uint32_t buf) {
        uint8_t* Ks = smem + buf * kStage;
        uint8_t* Vs = Ks + kKBytes;
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4*)(Ks + k_off(krow + 16u * i, kc)) = kr[i].f16();
        u32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = vr[i].f16();
        // keys 4*vkg..+3 = chunk c16 = vkg/4, group g = vkg%4 -> positions 16*c16 + vpos(4g)..+3
        const uint32_t pos = 16u * (vkg >> 2) + vpos(4u * (vkg & 3u));
        const uint32_t chunk = pos >> 3, sub = (pos & 7u) * 2u;  // byte offset inside the chunk
#pragma unroll
        for (int dd = 0; dd < 8; dd++) {
            const uint32_t w0 = v[0][dd >> 1], w1 = v[1][dd >> 1], w2 = v[2][dd >> 1], w3 = v[3][dd >> 1];
            const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
            u32x2 pr;
            pr.x = __builtin_amdgcn_perm(w1, w0, sel);
            pr.y = __builtin_amdgcn_perm(w3, w2, sel);
            const uint32_t d = 8u * vdg + dd;
            *(u32x2*)(Vs + v_off(d, chunk) + sub) = pr;
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 16; j++) o[i][j] = 0.0f;
    float m_i = -1.0e30f;  // running max, log2 domain (reference starts at -1e30)
    float l_i = 0.0f;      // this lane's partial row sum

    const uint32_t n_tiles = (S + kBKV - 1) / kBKV;
    load_tile(0);
    store_tile(0);
    __syncthreads();

    for (uint32_t t = 0; t < n_tiles; t++) {
        const uint32_t buf = t & 1u;
        if (t + 1 < n_tiles) load_tile(t + 1);
        const uint8_t* Ks = smem + buf * kStage;
        const uint8_t* Vs = Ks + kKBytes;

        // S^T[key][query] for the two 32-key halves of the tile
        f32x16 sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
#pragma unroll
            for (int j = 0; j < 16; j++) sacc[kb][j] = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    const f16x8 a = *(const f16x8*)(Ks + k_off(32u * kb + l32, 4u * c + 2u * kh + st));
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[c][st], sacc[kb], 0, 0, 0);
                }
        }
        // keys past the end contribute nothing (reference: score -1e30, p = 0)
        if ((t + 1) * kBKV > S) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const uint32_t key = t * kBKV + 32u * kb + 8u * (j >> 2) + 4u * kh + (j & 3);
                    if (key >= S) sacc[kb][j] = -INFINITY;
                }
        }
        float mx = sacc[0][0];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int j = 0; j < 16; j++) mx = fmaxf(mx, sacc[kb][j]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_i, mx * scale_log2);
        const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
        m_i = m_new;
        float rs = 0.0f;
        f16x8 pf[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][j], scale_log2, -m_new));
                rs += p;
                pf[kb][j >> 3][j & 7] = (_Float16)p;
            }
        l_i = l_i * alpha + rs;
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] *= alpha;

        // O^T[d][query] += V^T[d][key] P^T[key][query]
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const f16x8 a = *(const f16x8*)(Vs + v_off(32u * dt + l32, 2u * (2u * kb + c) + kh));
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[kb][c], o[dt], 0, 0, 0);
                }

        if (t + 1 < n_tiles) store_tile(buf ^ 1u);
        __syncthreads();
    }

    const float l_tot = l_i + __shfl_xor(l_i, 32);
    const float inv_l = 1.0f / l_tot;
    if (q_idx < S) {
        float* orow = O + (uint64_t)q_idx * H * kD + (uint64_t)head * kD;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t d = 32u * dt + 8u * g + 4u * kh;
                *(f32x4*)(orow + d) = f32x4{o[dt][4 * g] * inv_l, o[dt][4 * g + 1] * inv_l,
                                             o[dt][4 * g + 2] * inv_l, o[dt][4 * g + 3] * inv_l};
            }
    }
}

}  // namespace

hipError_t launch_flash_attention(const void* q, const void* k, const void* v, uint32_t xtype,
                                  float* o, uint32_t n_heads, uint32_t seq_len, float scale,
                                  hipStream_t st) {
    if (seq_len == 0 || n_heads == 0) return hipSuccess;
    const uint32_t n_qb = (seq_len + kBQ - 1) / kBQ;
    const dim3 grid(n_qb * n_heads);
    const float scale_log2 = scale * 1.4426950408889634f;
    switch (xtype) {
        case kGgmlF16:
            hipLaunchKernelGGL(flash_attn_fwd<kGgmlF16>, grid, dim3(256), 0, st, q, k, v, o, seq_len, n_heads,
                               scale_log2, n_qb);
            break;
        case kGgmlBF16:
            hipLaunchKernelGGL(flash_attn_fwd<kGgmlBF16>, grid, dim3(256), 0, st, q, k, v, o, seq_len, n_heads,
                               scale_log2, n_qb);
            break;
        default:
            hipLaunchKernelGGL(flash_attn_fwd<kGgmlF32>, grid, dim3(256), 0, st, q, k, v, o, seq_len, n_heads,
                               scale_log2, n_qb);
            break;
    }
    return hipGetLastError();
}

}  // namespace llmr
