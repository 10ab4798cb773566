/*
 * oracle.c - CPU restatement of llm-runner's DiT hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend. Loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the product.
 *
 * Built with -ffp-contract=off so every f32 operation rounds exactly where the
 * reference's source writes it. Where the reference leaves an order or a
 * contraction to its shader compiler, the choice made here is stated.
 *
 * Parity pins (checks that would catch a wrong restatement; tests/test_oracle_*.py):
 *   orc_f16_to_f32           exhaustive over all 65536 patterns vs numpy float16
 *                            widening, except exp=31 which must give +-Inf (the
 *                            reference's NaN->Inf quirk).
 *   orc_f32_to_f16           vs numpy float32->float16 (RNE) on 2^24 sampled
 *                            patterns plus every boundary/tie case.
 *   orc_f64_to_f16           vs numpy float64->float16 (one RNE rounding).
 *   orc_get_scale_min_k4     exhaustive over random 12-byte fields vs an
 *                            independent bit-field decoder + pack/unpack round trip.
 *   orc_dequant_q8_0         exhaustive: all 65536 scales x 256 int8 vs
 *                            numpy f32(d)*f32(q) (the product is exact in f32).
 *   orc_dequant_q8_0_operand exhaustive: all scales x all int8 vs numpy
 *                            float16 multiply (IEEE RNE).
 *   orc_dequant_q4k_operand  exact rational arithmetic (fractions) rounded to the
 *                            nearest half, ties to even, on blocks rich in ties.
 *   orc_dequant_q4k          exhaustive over (sc, mn, q) with special d/dmin
 *                            (0, subnormal, max, Inf) vs a float64 closed form
 *                            rounded once to f32.
 *   orc_quantize_q8_0        closed form in numpy float64 + float16 RNE; round
 *                            trip error <= d/2 per element.
 *   orc_quantize_q4k         own rule (no reference quantizer exists): checked
 *                            against the product's numpy quantizer byte for
 *                            byte and by the round-trip error bound.
 *   orc_batch_matmul_q8/q4k  float64 brute force on small shapes (tolerance
 *                            from the fp16 operand rounding), identity weights,
 *                            linearity in X, row_offset slicing == fused call.
 *   orc_batch_matmul_swiglu_q8  float64 brute force (dequantized weights,
 *                            silu(g) * u) on small shapes; gate/up swapped or
 *                            sigmoid-instead-of-silu restatements must fail it.
 *   orc_flash_attention      float64 textbook softmax attention on small shapes;
 *                            constant V -> O = V; S = 1 -> O = V; key permutation
 *                            invariance.
 *   orc_rope_tables/apply    closed form (cos/sin of pos*theta^(-2k/axis)) and
 *                            norm preservation of each rotated pair.
 *   orc_lora_down/up         integer operands (every sum exact) == int64
 *                            products with offsets; float data within f32
 *                            rounding of a float64 product.
 *   orc_q8_lora_merge        zero update == identity on reference-quantized
 *                            blocks; requantization error <= half a step plus
 *                            the f16 scale rounding; stored scale == f16 of
 *                            absmax/127; halves away from zero and saturation
 *                            on a hand-computed block; untouched rows.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------------------
 * fp16 <-> f32/f64
 * ------------------------------------------------------------------------- */

/* unpack_f16 (dependencies/llm_text.c3l/shaders/llm.slang:235-251) and
 * cpu_f16_to_f32 (lib/model/tensor.c3:130-147): exact for zero, subnormal and
 * normal halves; exponent 31 gives +-Inf for both Inf and NaN payloads. */
float orc_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exp_bits = (bits >> 10) & 0x1fu;
    uint32_t mant = bits & 0x3ffu;
    float val;
    if (exp_bits == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        val = ldexpf((float)mant, -24);
        return sign ? -val : val;
    }
    if (exp_bits == 31) return sign ? -INFINITY : INFINITY;
    val = ldexpf((float)(mant | 0x400u), (int)exp_bits - 25);
    return sign ? -val : val;
}

void orc_f16_to_f32_n(const uint16_t* bits, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(bits[i]);
}

/* Round-to-nearest-even binary32 -> binary16: Slang's float16_t(x), as used for
 * the activation tile (llm.slang:1673) and the FA tiles (flash_attn.slang:64). */
uint16_t orc_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> Inf */
    if (a >= 0x38800000u) {                                  /* normal half */
        uint32_t e16 = (a >> 23) - 112u;
        uint32_t mant = a & 0x7fffffu;
        uint32_t h = (e16 << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t e = a >> 23;
    if (e == 0) return sign; /* f32 zero/denormal: below half of 2^-24 */
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* value / 2^-24 = m * 2^(e-126) */
    if (shift > 24u) return sign;
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void orc_f32_to_f16_n(const float* x, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(x[i]);
}

/* binary64 -> binary16 with a single round-to-nearest-even, as CPython's
 * struct.pack('<e', d) does for the Q8_0 scale (tools/gguf_writer.py:141). */
uint16_t orc_f64_to_f16(double x) {
    uint64_t u;
    memcpy(&u, &x, 8);
    uint16_t sign = (uint16_t)((u >> 48) & 0x8000u);
    uint64_t a = u & 0x7fffffffffffffffull;
    if (a > 0x7ff0000000000000ull) return (uint16_t)(sign | 0x7e00u);
    double ax = fabs(x);
    if (ax >= 65520.0) return (uint16_t)(sign | 0x7c00u);
    uint64_t e = a >> 52;
    uint64_t mant = a & 0xfffffffffffffull;
    if (e >= 1009u) { /* >= 2^-14: normal half */
        uint64_t h = ((e - 1008u) << 10) | (mant >> 42);
        uint64_t rem = mant & ((1ull << 42) - 1u);
        uint64_t half = 1ull << 41;
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (e == 0) return sign;
    uint64_t m = mant | (1ull << 52);
    uint64_t shift = 1051u - e; /* value / 2^-24 = m * 2^(e-1051) */
    if (shift > 54u) return sign;
    uint64_t h = m >> shift;
    uint64_t rem = m & ((1ull << shift) - 1u);
    uint64_t half = 1ull << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---------------------------------------------------------------------------
 * GGUF block decode
 * ------------------------------------------------------------------------- */

/* get_scale_min_k4: llm.slang:447-462, identical to tensor.c3:304-317. */
void orc_get_scale_min_k4(uint32_t is, const uint8_t* s, uint32_t* sc, uint32_t* mn) {
    if (is < 4) {
        *sc = s[is] & 63u;
        *mn = s[is + 4] & 63u;
    } else {
        *sc = (s[is + 4] & 0xfu) | ((uint32_t)(s[is - 4] >> 6) << 4);
        *mn = (uint32_t)(s[is + 4] >> 4) | ((uint32_t)(s[is] >> 6) << 4);
    }
}

/* dequant_q8_0_block (lib/model/tensor.c3:354-361): out[i] = d * (float)qs[i]. */
void orc_dequant_q8_0(const uint8_t* blocks, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 34;
        float d = orc_f16_to_f32(rd_u16(blk));
        const int8_t* qs = (const int8_t*)(blk + 2);
        for (int i = 0; i < 32; i++) out[b * 32 + i] = d * (float)qs[i];
    }
}

/* batch_matmul_q8's B operand (llm.slang:1677-1705): the scale is stored as
 * float16_t(unpack_f16(bits)), each int8 as float16_t(q), and the two are
 * multiplied in fp16: RN16(d * q). d*q is exact in f32 (11 x 8 bits), so the
 * f32 product rounded once to fp16 is that fp16 multiply. */
void orc_dequant_q8_0_operand(const uint8_t* blocks, size_t nblocks, uint16_t* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 34;
        float s = orc_f16_to_f32(orc_f32_to_f16(orc_f16_to_f32(rd_u16(blk))));
        const int8_t* qs = (const int8_t*)(blk + 2);
        for (int i = 0; i < 32; i++) {
            float qh = orc_f16_to_f32(orc_f32_to_f16((float)qs[i]));
            out[b * 32 + i] = orc_f32_to_f16(s * qh);
        }
    }
}

/* dequant_q4k_block (lib/model/tensor.c3:292-335). Sub-block pair j covers
 * elements [64j, 64j+64): low nibbles of qs[32j..32j+31] with scale index 2j,
 * high nibbles with 2j+1. d*sc and dmin*mn are exact in f32, d*sc*q is exact,
 * so the single rounding is the subtraction, as on the GPU (llm.slang:2321-2328). */
void orc_dequant_q4k(const uint8_t* blocks, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 144;
        float* o = out + b * 256;
        float d = orc_f16_to_f32(rd_u16(blk));
        float dmin = orc_f16_to_f32(rd_u16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        for (uint32_t j = 0; j < 4; j++) {
            uint32_t sc1, m1, sc2, m2;
            orc_get_scale_min_k4(2 * j, scales, &sc1, &m1);
            orc_get_scale_min_k4(2 * j + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1, dm1 = dmin * (float)m1;
            float d2 = d * (float)sc2, dm2 = dmin * (float)m2;
            for (uint32_t l = 0; l < 32; l++) {
                uint32_t q = qs[j * 32 + l];
                o[j * 64 + l] = d1 * (float)(q & 0xfu) - dm1;
                o[j * 64 + 32 + l] = d2 * (float)((q >> 4) & 0xfu) - dm2;
            }
        }
    }
}

static double f16_value(uint16_t h) {
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    double v = e == 0 ? ldexp((double)m, -24) : ldexp((double)(m | 0x400u), (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}

/* binary16 nearest (ties to even) to the exact real a - b, for f32 a and b:
 * TwoSum gives hi + lo == a - b exactly; hi is rounded once, and when hi lies
 * exactly halfway between two halves a nonzero lo decides the direction. */
static uint16_t f16_of_exact_diff(float a, float b) {
    const double A = a, B = -(double)b;
    const double hi = A + B;
    const double bb = hi - A;
    const double lo = (A - (hi - bb)) + (B - bb);
    uint16_t h = orc_f64_to_f16(hi);
    if (lo == 0.0 || !isfinite(hi) || ((h & 0x7c00u) == 0x7c00u)) return h;
    const double hv = f16_value(h);
    /* the neighbour of h on the side of hi (in magnitude order within the sign) */
    uint16_t n;
    if (hi > hv)
        n = (h & 0x8000u) ? (uint16_t)(h == 0x8000u ? 0x0001u : h - 1u) : (uint16_t)(h + 1u);
    else if (hi < hv)
        n = (h & 0x8000u) ? (uint16_t)(h + 1u) : (uint16_t)(h == 0 ? 0x8001u : h - 1u);
    else
        return h; /* hi is a half: the residual cannot reach a rounding boundary */
    if ((n & 0x7c00u) == 0x7c00u) return h;
    if (hi != (hv + f16_value(n)) / 2) return h; /* not a tie */
    /* tie between h and n: the exact value lies on the side of lo */
    return ((lo > 0) == (f16_value(n) > hv)) ? n : h;
}

/* The Q4_K fp16 matrix operand: the exact value d*sc*q - dmin*mn (both
 * products exact in f32) rounded once to binary16 - what the gfx950 mixed
 * FMA (v_fma_mix{lo,hi}_f16) produces from the f32 operands. */
void orc_dequant_q4k_operand(const uint8_t* blocks, size_t nblocks, uint16_t* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 144;
        uint16_t* o = out + b * 256;
        float d = orc_f16_to_f32(rd_u16(blk));
        float dmin = orc_f16_to_f32(rd_u16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        for (uint32_t e = 0; e < 256; e++) {
            uint32_t j = e >> 6, h = (e >> 5) & 1u, l = e & 31u, sc, mn;
            orc_get_scale_min_k4(2 * j + h, scales, &sc, &mn);
            uint32_t q = (qs[j * 32 + l] >> (4 * h)) & 0xfu;
            float a = (d * (float)sc) * (float)q;
            float c = dmin * (float)mn;
            if (isnan(a) || isnan(c) || (isinf(a) && isinf(c) && a == c))
                o[e] = 0x7e00u;
            else
                o[e] = f16_of_exact_diff(a, c);
        }
    }
}

/* ---------------------------------------------------------------------------
 * Quantizers (input generation)
 * ------------------------------------------------------------------------- */

/* quantize_q8_0 (tools/gguf_writer.py:121-157): per 32-element block, in
 * double: amax = max|v|, d = amax/127 (1e-8 floor), scale stored with one RNE
 * rounding, q = floor(v/d + 0.5) (sign-symmetric: half away from zero) using
 * the unrounded d, clamped to [-127, 127]. */
void orc_quantize_q8_0(const float* x, size_t n, uint8_t* out) {
    size_t blocks = n / 32;
    for (size_t b = 0; b < blocks; b++) {
        const float* v = x + b * 32;
        double amax = 0.0;
        for (int i = 0; i < 32; i++) {
            double a = fabs((double)v[i]);
            if (a > amax) amax = a;
        }
        double d = amax / 127.0;
        if (d < 1e-8) d = 1e-8;
        double inv = 1.0 / d;
        uint8_t* blk = out + b * 34;
        uint16_t sb = orc_f64_to_f16(d);
        blk[0] = (uint8_t)(sb & 0xff);
        blk[1] = (uint8_t)(sb >> 8);
        for (int i = 0; i < 32; i++) {
            double vi = (double)v[i];
            double q = vi >= 0 ? floor(vi * inv + 0.5) : -floor(-vi * inv + 0.5);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            blk[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

static double clampd(double v, double lo, double hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* The build's own Q4_K rule (no reference quantizer exists). Per 256-element
 * superblock, in double: for each 32-element sub-block s, mn_s = max(0, -min),
 * sc_s = (max + mn_s)/15; d = max(sc)/63, dmin = max(mn)/63 stored as RNE
 * halves; 6-bit ls = round(sc_s/d), lm = round(mn_s/dmin); q = round((v +
 * dmin*lm)/(d*ls)) clamped to [0,15]; round(x) = floor(x + 0.5). Packing is the
 * inverse of get_scale_min_k4 and of the nibble layout of tensor.c3:319-331. */
void orc_quantize_q4k(const float* x, size_t n, uint8_t* out) {
    size_t blocks = n / 256;
    for (size_t b = 0; b < blocks; b++) {
        const float* v = x + b * 256;
        double sc[8], mn[8];
        double dmax = 0.0, mmax = 0.0;
        for (int s = 0; s < 8; s++) {
            double lo = (double)v[32 * s], hi = lo;
            for (int l = 1; l < 32; l++) {
                double t = (double)v[32 * s + l];
                if (t < lo) lo = t;
                if (t > hi) hi = t;
            }
            mn[s] = lo < 0 ? -lo : 0.0;
            sc[s] = (hi + mn[s]) / 15.0;
            if (sc[s] > dmax) dmax = sc[s];
            if (mn[s] > mmax) mmax = mn[s];
        }
        uint16_t dbits = orc_f64_to_f16(dmax / 63.0);
        uint16_t mbits = orc_f64_to_f16(mmax / 63.0);
        double dd = (double)orc_f16_to_f32(dbits);
        double dm = (double)orc_f16_to_f32(mbits);
        uint32_t ls[8], lm[8];
        uint8_t q[256];
        for (int s = 0; s < 8; s++) {
            ls[s] = dd > 0 ? (uint32_t)clampd(floor(sc[s] / dd + 0.5), 0, 63) : 0;
            lm[s] = dm > 0 ? (uint32_t)clampd(floor(mn[s] / dm + 0.5), 0, 63) : 0;
            double S = dd * (double)ls[s];
            double O = dm * (double)lm[s];
            for (int l = 0; l < 32; l++) {
                double t = (double)v[32 * s + l];
                q[32 * s + l] = S > 0 ? (uint8_t)clampd(floor((t + O) / S + 0.5), 0, 15) : 0;
            }
        }
        uint8_t* blk = out + b * 144;
        blk[0] = (uint8_t)(dbits & 0xff);
        blk[1] = (uint8_t)(dbits >> 8);
        blk[2] = (uint8_t)(mbits & 0xff);
        blk[3] = (uint8_t)(mbits >> 8);
        uint8_t* s12 = blk + 4;
        for (int j = 0; j < 4; j++) {
            s12[j] = (uint8_t)((ls[j] & 63u) | ((ls[j + 4] >> 4) << 6));
            s12[j + 4] = (uint8_t)((lm[j] & 63u) | ((lm[j + 4] >> 4) << 6));
            s12[j + 8] = (uint8_t)((ls[j + 4] & 15u) | ((lm[j + 4] & 15u) << 4));
        }
        uint8_t* qs = blk + 16;
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++)
                qs[32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
    }
}

/* ---------------------------------------------------------------------------
 * GEMMs
 * ------------------------------------------------------------------------- */

#define ORC_NB 32 /* output columns per work item: independent f32 chains */

/* batch_matmul_q8 (llm.slang:1613-1767), restricted to output rows `rows`.
 * Per output: acc = 0; for t in 0..K/32-1: for kp in 0..15:
 *   acc += a.x*b.x + a.y*b.y     (a = fp16(x), b = RN16(d*q))
 * The two products are exact in f32 (fp16 x fp16), so whether the shader
 * compiler contracts them into an FMA does not change the result. */
void orc_batch_matmul_q8_rows(const uint8_t* W, const float* X, float* Y, uint32_t N, uint32_t K,
                              uint32_t M, uint32_t row_offset, const uint32_t* rows,
                              uint32_t n_rows) {
    (void)M;
    const size_t bpr = K / 32;
    /* activations rounded to fp16 once */
    float* A = (float*)malloc(sizeof(float) * (size_t)n_rows * K);
    for (uint32_t r = 0; r < n_rows; r++)
        for (uint32_t k = 0; k < K; k++)
            A[(size_t)r * K + k] = orc_f16_to_f32(orc_f32_to_f16(X[(size_t)rows[r] * K + k]));
    uint32_t nblk = (N + ORC_NB - 1) / ORC_NB;
#pragma omp parallel for schedule(dynamic)
    for (uint32_t jb = 0; jb < nblk; jb++) {
        uint32_t n0 = jb * ORC_NB;
        uint32_t nn = N - n0 < ORC_NB ? N - n0 : ORC_NB;
        /* B^T block [K][ORC_NB] of fp16 operand values */
        float* BT = (float*)calloc((size_t)K * ORC_NB, sizeof(float));
        uint16_t* tmp = (uint16_t*)malloc(sizeof(uint16_t) * K);
        for (uint32_t j = 0; j < nn; j++) {
            const uint8_t* wrow = W + (size_t)(row_offset + n0 + j) * bpr * 34;
            orc_dequant_q8_0_operand(wrow, bpr, tmp);
            for (uint32_t k = 0; k < K; k++) BT[(size_t)k * ORC_NB + j] = orc_f16_to_f32(tmp[k]);
        }
        float acc[ORC_NB];
        for (uint32_t r = 0; r < n_rows; r++) {
            const float* a = A + (size_t)r * K;
            for (int j = 0; j < ORC_NB; j++) acc[j] = 0.0f;
            for (uint32_t k = 0; k < K; k += 2) {
                const float ax = a[k], ay = a[k + 1];
                const float* b0 = BT + (size_t)k * ORC_NB;
                const float* b1 = b0 + ORC_NB;
                for (int j = 0; j < ORC_NB; j++) acc[j] += ax * b0[j] + ay * b1[j];
            }
            for (uint32_t j = 0; j < nn; j++) Y[(size_t)r * N + n0 + j] = acc[j];
        }
        free(tmp);
        free(BT);
    }
    free(A);
}

void orc_batch_matmul_q8(const uint8_t* W, const float* X, float* Y, uint32_t N, uint32_t K,
                         uint32_t M, uint32_t row_offset) {
    uint32_t* rows = (uint32_t*)malloc(sizeof(uint32_t) * (M ? M : 1));
    for (uint32_t i = 0; i < M; i++) rows[i] = i;
    orc_batch_matmul_q8_rows(W, X, Y, N, K, M, row_offset, rows, M);
    free(rows);
}

/* batch_matmul_swiglu_q8 (llm.slang:1769-1911), restricted to output rows
 * `rows`. Unlike batch_matmul_q8 everything is f32: the activations are not
 * rounded and the weight is dequant_q8_at = f32(d) * q (llm.slang:1797-1813,
 * exact in f32). Per output: g = u = 0; for t in 0..K/32-1: for k in 0..31:
 *   g += a_k * bg_k;  u += a_k * bu_k       (one rounding per mul and add here;
 * the reference leaves contraction of these to its shader compiler, so an
 * FMA there differs by an ulp per step, far inside the GEMM tolerance)
 * then out = silu(g) * u with silu(g) = g / (1 + exp(-g)) (llm.slang:1901-1904). */
void orc_batch_matmul_swiglu_q8_rows(const uint8_t* Wg, const uint8_t* Wu, const float* X, float* Y,
                                     uint32_t N, uint32_t K, uint32_t M, const uint32_t* rows,
                                     uint32_t n_rows) {
    (void)M;
    const size_t bpr = K / 32;
    uint32_t nblk = (N + ORC_NB - 1) / ORC_NB;
#pragma omp parallel for schedule(dynamic)
    for (uint32_t jb = 0; jb < nblk; jb++) {
        uint32_t n0 = jb * ORC_NB;
        uint32_t nn = N - n0 < ORC_NB ? N - n0 : ORC_NB;
        float* BG = (float*)calloc((size_t)K * ORC_NB, sizeof(float));
        float* BU = (float*)calloc((size_t)K * ORC_NB, sizeof(float));
        float* tmp = (float*)malloc(sizeof(float) * K);
        for (uint32_t j = 0; j < nn; j++) {
            orc_dequant_q8_0(Wg + (size_t)(n0 + j) * bpr * 34, bpr, tmp);
            for (uint32_t k = 0; k < K; k++) BG[(size_t)k * ORC_NB + j] = tmp[k];
            orc_dequant_q8_0(Wu + (size_t)(n0 + j) * bpr * 34, bpr, tmp);
            for (uint32_t k = 0; k < K; k++) BU[(size_t)k * ORC_NB + j] = tmp[k];
        }
        float g[ORC_NB], u[ORC_NB];
        for (uint32_t r = 0; r < n_rows; r++) {
            const float* a = X + (size_t)rows[r] * K;
            for (int j = 0; j < ORC_NB; j++) g[j] = u[j] = 0.0f;
            for (uint32_t k = 0; k < K; k++) {
                const float ak = a[k];
                const float* bg = BG + (size_t)k * ORC_NB;
                const float* bu = BU + (size_t)k * ORC_NB;
                for (int j = 0; j < ORC_NB; j++) {
                    g[j] += ak * bg[j];
                    u[j] += ak * bu[j];
                }
            }
            for (uint32_t j = 0; j < nn; j++) {
                const float silu = g[j] / (1.0f + expf(-g[j]));
                Y[(size_t)r * N + n0 + j] = silu * u[j];
            }
        }
        free(tmp);
        free(BU);
        free(BG);
    }
}

void orc_batch_matmul_swiglu_q8(const uint8_t* Wg, const uint8_t* Wu, const float* X, float* Y, uint32_t N,
                                uint32_t K, uint32_t M) {
    uint32_t* rows = (uint32_t*)malloc(sizeof(uint32_t) * (M ? M : 1));
    for (uint32_t i = 0; i < M; i++) rows[i] = i;
    orc_batch_matmul_swiglu_q8_rows(Wg, Wu, X, Y, N, K, M, rows, M);
    free(rows);
}

/* batch_matmul_q4k (llm.slang:2264-2365), restricted to output rows `rows`.
 * Operands stay f32: a = x, b = d*sc*q - dmin*mn; acc += a*b with k ascending
 * (K-tile t, then k_local 0..31). Whether the shader compiler contracts
 * acc += a*b into an FMA is unspecified by the source; this restatement
 * rounds the product and the sum separately. */
void orc_batch_matmul_q4k_rows(const uint8_t* W, const float* X, float* Y, uint32_t N,
                               uint32_t K, uint32_t M, uint32_t row_offset,
                               const uint32_t* rows, uint32_t n_rows) {
    (void)M;
    const size_t bpr = K / 256;
    uint32_t nblk = (N + ORC_NB - 1) / ORC_NB;
#pragma omp parallel for schedule(dynamic)
    for (uint32_t jb = 0; jb < nblk; jb++) {
        uint32_t n0 = jb * ORC_NB;
        uint32_t nn = N - n0 < ORC_NB ? N - n0 : ORC_NB;
        float* BT = (float*)calloc((size_t)K * ORC_NB, sizeof(float));
        float* tmp = (float*)malloc(sizeof(float) * K);
        for (uint32_t j = 0; j < nn; j++) {
            const uint8_t* wrow = W + (size_t)(row_offset + n0 + j) * bpr * 144;
            orc_dequant_q4k(wrow, bpr, tmp);
            for (uint32_t k = 0; k < K; k++) BT[(size_t)k * ORC_NB + j] = tmp[k];
        }
        float acc[ORC_NB];
        for (uint32_t r = 0; r < n_rows; r++) {
            const float* a = X + (size_t)rows[r] * K;
            for (int j = 0; j < ORC_NB; j++) acc[j] = 0.0f;
            for (uint32_t k = 0; k < K; k++) {
                const float ak = a[k];
                const float* b = BT + (size_t)k * ORC_NB;
                for (int j = 0; j < ORC_NB; j++) acc[j] += ak * b[j];
            }
            for (uint32_t j = 0; j < nn; j++) Y[(size_t)r * N + n0 + j] = acc[j];
        }
        free(tmp);
        free(BT);
    }
}

void orc_batch_matmul_q4k(const uint8_t* W, const float* X, float* Y, uint32_t N, uint32_t K,
                          uint32_t M, uint32_t row_offset) {
    uint32_t* rows = (uint32_t*)malloc(sizeof(uint32_t) * (M ? M : 1));
    for (uint32_t i = 0; i < M; i++) rows[i] = i;
    orc_batch_matmul_q4k_rows(W, X, Y, N, K, M, row_offset, rows, M);
    free(rows);
}

/* ---------------------------------------------------------------------------
 * Flash attention (flash_attn.slang:38-241)
 * ------------------------------------------------------------------------- */

#define FA_BR 16
#define FA_BC 32

static inline float rnd16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

void orc_flash_attention(const float* Q, const float* K, const float* V, float* O, uint32_t D,
                         uint32_t H, uint32_t S, float scale, uint32_t h0, uint32_t h1,
                         uint32_t q0, uint32_t q1) {
    if (D != 128 || h1 <= h0 || q1 <= q0) return;
    uint32_t qb0 = q0 / FA_BR, qb1 = (q1 + FA_BR - 1) / FA_BR;
    uint32_t nqb = qb1 - qb0;
    uint32_t n_items = (h1 - h0) * nqb;
    const uint32_t n_kv_blocks = (S + FA_BC - 1) / FA_BC;
    const size_t dim = (size_t)H * D;
#pragma omp parallel for schedule(dynamic)
    for (uint32_t item = 0; item < n_items; item++) {
        uint32_t head = h0 + item / nqb;
        uint32_t q_start = (qb0 + item % nqb) * FA_BR;
        size_t ho = (size_t)head * S * D;
        float Qt[FA_BR][128], Kt[FA_BC][128], Sx[FA_BR][FA_BC];
        float m[FA_BR], l[FA_BR], acc[FA_BR][128];
        for (uint32_t r = 0; r < FA_BR; r++) {
            uint32_t aq = q_start + r;
            for (uint32_t d = 0; d < 128; d++) {
                Qt[r][d] = aq < S ? rnd16(Q[ho + (size_t)aq * D + d]) : 0.0f;
                acc[r][d] = 0.0f;
            }
            m[r] = -1.0e30f;
            l[r] = 0.0f;
        }
        for (uint32_t kb = 0; kb < n_kv_blocks; kb++) {
            uint32_t kv_start = kb * FA_BC;
            /* 3a: K tile (fp16) */
            for (uint32_t c = 0; c < FA_BC; c++) {
                uint32_t ak = kv_start + c;
                for (uint32_t d = 0; d < 128; d++)
                    Kt[c][d] = ak < S ? rnd16(K[ho + (size_t)ak * D + d]) : 0.0f;
            }
            /* 3b: scores, dot over half2 pairs in order dp = 0..63 */
            for (uint32_t r = 0; r < FA_BR; r++)
                for (uint32_t c = 0; c < FA_BC; c++) {
                    float dot = 0.0f;
                    for (uint32_t dp = 0; dp < 64; dp++)
                        dot += Qt[r][2 * dp] * Kt[c][2 * dp] + Qt[r][2 * dp + 1] * Kt[c][2 * dp + 1];
                    dot *= scale;
                    int valid = (kv_start + c < S) && (q_start + r < S);
                    Sx[r][c] = valid ? dot : -1.0e30f;
                }
            /* 3c-3d: row max, exp, tree-reduced row sum, running state */
            float rescale[FA_BR];
            for (uint32_t r = 0; r < FA_BR; r++) {
                float red[FA_BC];
                for (uint32_t c = 0; c < FA_BC; c++) red[c] = Sx[r][c];
                for (uint32_t s = 16; s > 0; s >>= 1)
                    for (uint32_t c = 0; c < s; c++) red[c] = fmaxf(red[c], red[c + s]);
                float m_new = fmaxf(m[r], red[0]);
                for (uint32_t c = 0; c < FA_BC; c++) {
                    int valid = (kv_start + c < S) && (q_start + r < S);
                    Sx[r][c] = valid ? expf(Sx[r][c] - m_new) : 0.0f;
                    red[c] = Sx[r][c];
                }
                for (uint32_t s = 16; s > 0; s >>= 1)
                    for (uint32_t c = 0; c < s; c++) red[c] += red[c + s];
                float rv = expf(m[r] - m_new);
                m[r] = m_new;
                l[r] = rv * l[r] + red[0];
                rescale[r] = rv;
            }
            /* 3e-3f: V tile (fp16, reusing Kt), O = rescale*O + P@V */
            for (uint32_t c = 0; c < FA_BC; c++) {
                uint32_t ak = kv_start + c;
                for (uint32_t d = 0; d < 128; d++)
                    Kt[c][d] = ak < S ? rnd16(V[ho + (size_t)ak * D + d]) : 0.0f;
            }
            for (uint32_t r = 0; r < FA_BR; r++)
                for (uint32_t d = 0; d < 128; d++) {
                    float nv = 0.0f;
                    for (uint32_t c = 0; c < FA_BC; c++) nv += Sx[r][c] * Kt[c][d];
                    acc[r][d] = acc[r][d] * rescale[r] + nv;
                }
        }
        /* step 4: normalise with the reciprocal, fused reverse transpose */
        for (uint32_t r = 0; r < FA_BR; r++) {
            uint32_t aq = q_start + r;
            if (aq >= S || aq < q0 || aq >= q1) continue;
            float inv_l = 1.0f / l[r];
            for (uint32_t d = 0; d < 128; d++)
                O[(size_t)aq * dim + (size_t)head * D + d] = acc[r][d] * inv_l;
        }
    }
}

/* ---------------------------------------------------------------------------
 * RoPE (input preparation for attention)
 * ------------------------------------------------------------------------- */

/* precompute_flux_mrope (dependencies/flux.c3l/flux_dit.c3:396-529) with the
 * axis list as a parameter: pair index runs over the axes in order; within
 * axis a of size dims_a, pair k uses freq = 1/theta^(2k/dims_a) and angle =
 * pos_a * freq, all in f32. */
void orc_rope_tables(const uint32_t* pos, uint32_t S, const uint32_t* axes_dims, uint32_t n_axes,
                     float theta, float* cos_out, float* sin_out) {
    for (uint32_t t = 0; t < S; t++) {
        uint32_t pair = 0;
        for (uint32_t a = 0; a < n_axes; a++) {
            uint32_t half_ax = axes_dims[a] / 2;
            for (uint32_t k = 0; k < half_ax; k++) {
                float freq = 1.0f / powf(theta, (float)(2 * k) / (float)axes_dims[a]);
                float angle = (float)pos[(size_t)t * n_axes + a] * freq;
                cos_out[(size_t)t * 64 + pair] = cosf(angle);
                sin_out[(size_t)t * 64 + pair] = sinf(angle);
                pair++;
            }
        }
    }
}

/* mrope (dependencies/zimage.c3l/shaders/mrope.slang:33-54): interleaved pairs,
 * x0' = x0*c - x1*s, x1' = x0*s + x1*c, on [H, S, 128]. */
void orc_rope_apply(float* x, uint32_t H, uint32_t S, const float* cos_t, const float* sin_t) {
    for (uint32_t h = 0; h < H; h++)
        for (uint32_t p = 0; p < S; p++) {
            float* row = x + ((size_t)h * S + p) * 128;
            for (uint32_t j = 0; j < 64; j++) {
                float c = cos_t[(size_t)p * 64 + j], s = sin_t[(size_t)p * 64 + j];
                float x0 = row[2 * j], x1 = row[2 * j + 1];
                row[2 * j] = x0 * c - x1 * s;
                row[2 * j + 1] = x0 * s + x1 * c;
            }
        }
}

/* ---------------------------------------------------------------------------
 * DiT block glue (the dispatches between the GEMMs and attention), each as
 * its own op exactly as the reference dispatches it, f32, in place where the
 * reference works in place.
 * ------------------------------------------------------------------------- */

/* The shared-memory reduction of a 256-thread workgroup: thread gi first sums
 * its strided elements in order (i = gi, gi+256, ...), then the tree
 * s = 128, 64, ..., 1: part[gi] += part[gi + s]. */
static float wg_tree_sum(float part[256]) {
    for (uint32_t s = 128; s > 0; s >>= 1)
        for (uint32_t gi = 0; gi < s; gi++) part[gi] += part[gi + s];
    return part[0];
}

/* batch_rmsnorm (zimage.slang:449-500): out = x * (1/sqrt(sum/dim + eps)) * w. */
void orc_batch_rmsnorm(const float* x, const float* w, float* out, uint32_t dim, uint32_t n_rows, float eps) {
#pragma omp parallel for schedule(static)
    for (uint32_t r = 0; r < n_rows; r++) {
        const float* xr = x + (size_t)r * dim;
        float part[256];
        for (uint32_t gi = 0; gi < 256; gi++) {
            float s = 0.0f;
            for (uint32_t i = gi; i < dim; i += 256) s += xr[i] * xr[i];
            part[gi] = s;
        }
        float rms = 1.0f / sqrtf(wg_tree_sum(part) / (float)dim + eps);
        for (uint32_t i = 0; i < dim; i++) out[(size_t)r * dim + i] = xr[i] * rms * w[i];
    }
}

/* batch_layernorm (zimage.slang:502-561): two passes, no affine. */
void orc_batch_layernorm(const float* x, float* out, uint32_t dim, uint32_t n_rows, float eps) {
#pragma omp parallel for schedule(static)
    for (uint32_t r = 0; r < n_rows; r++) {
        const float* xr = x + (size_t)r * dim;
        float part[256];
        for (uint32_t gi = 0; gi < 256; gi++) {
            float s = 0.0f;
            for (uint32_t i = gi; i < dim; i += 256) s += xr[i];
            part[gi] = s;
        }
        float mean = wg_tree_sum(part) / (float)dim;
        for (uint32_t gi = 0; gi < 256; gi++) {
            float s = 0.0f;
            for (uint32_t i = gi; i < dim; i += 256) {
                float d = xr[i] - mean;
                s += d * d;
            }
            part[gi] = s;
        }
        float inv_std = 1.0f / sqrtf(wg_tree_sum(part) / (float)dim + eps);
        for (uint32_t i = 0; i < dim; i++) out[(size_t)r * dim + i] = (xr[i] - mean) * inv_std;
    }
}

/* scale_modulate (zimage.slang:356-373): x[i] = x[i] * (1 + scale[i % dim]), and
 * adaln_modulate (zimage.slang:98-117): x[i] = x[i] * (1 + scale[d]) + shift[d];
 * shift == NULL selects the former. In place over n elements. */
void orc_modulate(float* x, const float* scale, const float* shift, uint32_t dim, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint32_t d = (uint32_t)(i % dim);
        x[i] = shift ? x[i] * (1.0f + scale[d]) + shift[d] : x[i] * (1.0f + scale[d]);
    }
}

/* batch_head_norm (zimage.slang:609-667): per (pos, head) RMSNorm over D, in place. */
void orc_batch_head_norm(float* x, const float* w, uint32_t n_heads, uint32_t D, uint32_t seq_len, float eps) {
#pragma omp parallel for schedule(static)
    for (uint32_t g = 0; g < seq_len * n_heads; g++) {
        float* row = x + (size_t)g * D;
        float part[256];
        for (uint32_t gi = 0; gi < 256; gi++) {
            float s = 0.0f;
            for (uint32_t i = gi; i < D; i += 256) s += row[i] * row[i];
            part[gi] = s;
        }
        float rms = 1.0f / sqrtf(wg_tree_sum(part) / (float)D + eps);
        for (uint32_t i = 0; i < D; i++) row[i] = row[i] * rms * w[i];
    }
}

/* transpose_heads direction 0 (zimage.slang:563-601): [S, H, D] -> [H, S, D]. */
void orc_transpose_heads(const float* in, float* out, uint32_t S, uint32_t H, uint32_t D) {
    for (uint32_t s = 0; s < S; s++)
        for (uint32_t h = 0; h < H; h++)
            memcpy(out + ((size_t)h * S + s) * D, in + ((size_t)s * H + h) * D, D * sizeof(float));
}

/* gated_residual (zimage.slang:382-410) with scale <= 0 -> 1 and clip <= 0 ->
 * 1e10, and gated_residual_linear (zimage.slang:414-424) when tanh_gate == 0:
 * residual[i] += g(d) * input[i], d = i % dim. */
void orc_gated_residual(float* residual, const float* gate, const float* input, uint32_t dim, size_t n,
                        int tanh_gate, float scale, float clip_thresh) {
    float rs = scale > 0.0f ? scale : 1.0f;
    float ct = clip_thresh > 0.0f ? clip_thresh : 1e10f;
    for (size_t i = 0; i < n; i++) {
        uint32_t d = (uint32_t)(i % dim);
        if (tanh_gate) {
            float v = rs * tanhf(gate[d]) * input[i];
            v = v < -ct ? -ct : (v > ct ? ct : v);
            residual[i] += v;
        } else {
            residual[i] += gate[d] * input[i];
        }
    }
}

/* silu (diffusion.slang:1082-1086), gelu (tanh form, diffusion.slang:1092-1107),
 * in place over n elements. */
void orc_silu(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}
void orc_gelu(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        float c = 0.7978845608f;
        x[i] = 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
    }
}

/* dit_timestep_embed (zimage.slang:284-307). */
void orc_timestep_embed(float* out, uint32_t dim, float t) {
    uint32_t half = dim / 2;
    for (uint32_t i = 0; i < dim; i++) {
        uint32_t j = i < half ? i : i - half;
        float freq = expf(-logf(10000.0f) * (float)j / (float)half);
        out[i] = i < half ? cosf(t * freq) : sinf(t * freq);
    }
}

/* patchify (zimage.slang:11-51): [C, H, W] -> [n_patches, C*ps*ps]. */
void orc_patchify(const float* in, float* out, uint32_t C, uint32_t H, uint32_t W, uint32_t ps) {
    uint32_t pd = C * ps * ps, pw = W / ps, n = (H / ps) * pw * pd;
    for (uint32_t t = 0; t < n; t++) {
        uint32_t p = t / pd, e = t % pd;
        uint32_t py = e / (ps * C), px = (e % (ps * C)) / C, c = e % C;
        uint32_t ih = (p / pw) * ps + py, iw = (p % pw) * ps + px;
        out[t] = in[(size_t)c * H * W + (size_t)ih * W + iw];
    }
}

/* unpatchify (zimage.slang:56-93): [n_patches, C*ps*ps] -> [C, H, W]. */
void orc_unpatchify(const float* in, float* out, uint32_t C, uint32_t H, uint32_t W, uint32_t ps) {
    for (uint32_t t = 0; t < C * H * W; t++) {
        uint32_t c = t / (H * W), rem = t % (H * W), h = rem / W, w = rem % W;
        uint32_t p = (h / ps) * (W / ps) + w / ps;
        uint32_t e = (h % ps) * ps * C + (w % ps) * C + c;
        out[t] = in[(size_t)p * C * ps * ps + e];
    }
}

/* ---- LoRA (dispatch_lora_correction, dit.c3:1319-1364; q8_lora_merge) ----
 * The reference's `partial += a * b` dot products leave contraction to the
 * Vulkan driver (its SPIR-V carries no NoContraction); here they are fused
 * multiply-adds (fmaf), the matrix math's one contraction. Every other
 * expression rounds each operation. */

/* Hop 1: batch_matmul_simple (llm.slang:1146-1180) with the LoRA A [rank,
 * in_dim] as its weight: scratch[s, r] = sum_k A[r, k] * x[s, k], each sum
 * formed as one 256-thread workgroup forms it: fused partials, then
 * wg_tree_sum. */
void orc_lora_down(const float* A, const float* X, float* scratch, uint32_t rank, uint32_t in_dim,
                   uint32_t seq_len) {
#pragma omp parallel for schedule(static)
    for (int64_t sr = 0; sr < (int64_t)seq_len * rank; sr++) {
        const uint32_t s = (uint32_t)(sr / rank), r = (uint32_t)(sr % rank);
        float part[256];
        for (uint32_t gi = 0; gi < 256; gi++) {
            float p = 0.0f;
            for (uint32_t k = gi; k < in_dim; k += 256) p = fmaf(A[(size_t)r * in_dim + k], X[(size_t)s * in_dim + k], p);
            part[gi] = p;
        }
        scratch[sr] = wg_tree_sum(part);
    }
}

/* Hop 2: batch_matmul_add_scaled (llm.slang:1262-1294): for o < b_rows,
 * out[s * out_dim + row_offset + o] += scale * (fused sum over r in order of
 * B[(weight_row_offset + o) * rank + r] * scratch[s * rank + r]). */
void orc_lora_up(const float* B, const float* scratch, float* out, uint32_t rank, uint32_t out_dim,
                 uint32_t seq_len, float scale, uint32_t row_offset, uint32_t weight_row_offset, uint32_t b_rows) {
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < (int64_t)seq_len; s++)
        for (uint32_t o = 0; o < b_rows; o++) {
            const float* b = B + (size_t)(weight_row_offset + o) * rank;
            float p = 0.0f;
            for (uint32_t r = 0; r < rank; r++) p = fmaf(b[r], scratch[(size_t)s * rank + r], p);
            float* y = out + (size_t)s * out_dim + row_offset + o;
            *y = *y + scale * p;
        }
}

/* q8_lora_merge (llm.slang:1337-1420), in place on rows [dst_row_offset,
 * dst_row_offset + b_rows) of a Q8_0 weight (in_dim % 256 == 0): element k
 * of LoRA row j becomes d * q + scale * (fused sum over r in order of B[j, r] *
 * A[r, k]); each 32-element block is requantized with d' = max(absmax / 127,
 * 1e-8) (f32), q' = clamp(trunc(u / d' +- 0.5), -127, 127) (the half added
 * in f32), and d' stored as f16 (round to nearest even). */
void orc_q8_lora_merge(uint8_t* base, const float* A, const float* B, uint32_t in_dim, uint32_t b_rows,
                       uint32_t dst_row_offset, uint32_t rank, float scale) {
    const size_t row_bytes = (size_t)(in_dim / 32) * 34;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < (int64_t)b_rows; j++) {
        uint8_t* row = base + (size_t)(dst_row_offset + (uint32_t)j) * row_bytes;
        for (uint32_t blk = 0; blk < in_dim / 32; blk++) {
            uint8_t* b = row + (size_t)blk * 34;
            const float d = orc_f16_to_f32(rd_u16(b));
            float u[32], amax = 0.0f;
            for (uint32_t i = 0; i < 32; i++) {
                const uint32_t k = blk * 32 + i;
                const float base_val = d * (float)(int8_t)b[2 + i];
                float delta = 0.0f;
                for (uint32_t r = 0; r < rank; r++) delta = fmaf(B[(size_t)j * rank + r], A[(size_t)r * in_dim + k], delta);
                delta *= scale;
                u[i] = base_val + delta;
                const float a = fabsf(u[i]);
                if (a > amax) amax = a;
            }
            float dn = amax / 127.0f;
            if (dn < 1e-8f) dn = 1e-8f;
            for (uint32_t i = 0; i < 32; i++) {
                const float qf = u[i] / dn;
                int q = qf >= 0.0f ? (int)(qf + 0.5f) : (int)(qf - 0.5f);
                q = q < -127 ? -127 : (q > 127 ? 127 : q);
                b[2 + i] = (uint8_t)(int8_t)q;
            }
            const uint16_t h = orc_f32_to_f16(dn);
            b[0] = (uint8_t)(h & 0xffu);
            b[1] = (uint8_t)(h >> 8);
        }
    }
}
