/*
 * oracle.h - CPU restatement of llm-runner's DiT hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP backend:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The product (llm-runner_amd/) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the llm-runner tree). Parity pins (what checks each function beyond its own
 * formula) are listed in oracle.c's header comment.
 */
#ifndef LLMR_ORACLE_H
#define LLMR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 decode: unpack_f16 (llm.slang:235-251) == cpu_f16_to_f32 (tensor.c3:130-147). */
float orc_f16_to_f32(uint16_t bits);
void orc_f16_to_f32_n(const uint16_t* bits, size_t n, float* out);

/* IEEE binary32 -> binary16, round to nearest even (Slang float16_t(x)). */
uint16_t orc_f32_to_f16(float x);
void orc_f32_to_f16_n(const float* x, size_t n, uint16_t* out);

/* IEEE binary64 -> binary16, round to nearest even, one rounding
 * (Python struct '<e', used by gguf_writer.py:141). */
uint16_t orc_f64_to_f16(double x);

/* get_scale_min_k4 (llm.slang:447-462 == tensor.c3:304-317). */
void orc_get_scale_min_k4(uint32_t is, const uint8_t* scales12, uint32_t* sc, uint32_t* mn);

/* CPU dequant (tensor.c3:354-361, tensor.c3:292-335): nblocks blocks -> f32. */
void orc_dequant_q8_0(const uint8_t* blocks, size_t nblocks, float* out);
void orc_dequant_q4k(const uint8_t* blocks, size_t nblocks, float* out);

/* The fp16 matrix operand of batch_matmul_q8 (llm.slang:1677-1705):
 * RN16(fp16(unpack_f16(d)) * fp16(q)). */
void orc_dequant_q8_0_operand(const uint8_t* blocks, size_t nblocks, uint16_t* out);

/* The Q4_K fp16 matrix operand: the exact d*sc*q - dmin*mn rounded once to
 * binary16 (the f32 value of tensor.c3:319-331 before its own rounding). */
void orc_dequant_q4k_operand(const uint8_t* blocks, size_t nblocks, uint16_t* out);

/* Q8_0 quantizer of tools/gguf_writer.py:121-157 (double math, RNE scale). */
void orc_quantize_q8_0(const float* x, size_t n, uint8_t* out);

/* Q4_K quantizer. The reference has none (gguf_writer.py:51-60,160-169 stop at
 * Q8_0); this is the build's own rule, restated here so the product's numpy
 * quantizer can be checked byte for byte. */
void orc_quantize_q4k(const float* x, size_t n, uint8_t* out);

/* batch_matmul_q8 (llm.slang:1613-1767): a = fp16(x), b = RN16(d*q),
 * acc += a.x*b.x + a.y*b.y over t = 0..K/32-1, kp = 0..15.
 * W: raw Q8_0 tensor, rows [row_offset, row_offset+N); X f32 [M,K]; Y f32 [M,N]. */
void orc_batch_matmul_q8(const uint8_t* W, const float* X, float* Y, uint32_t N, uint32_t K,
                         uint32_t M, uint32_t row_offset);

/* batch_matmul_q4k (llm.slang:2264-2365): all f32, acc += a*b over k in order. */
void orc_batch_matmul_q4k(const uint8_t* W, const float* X, float* Y, uint32_t N, uint32_t K,
                          uint32_t M, uint32_t row_offset);

/* Same GEMMs restricted to the output rows listed in `rows` (indices into M);
 * Y is [n_rows, N]. Used to check full-size launches on a sample of tokens. */
void orc_batch_matmul_q8_rows(const uint8_t* W, const float* X, float* Y, uint32_t N, uint32_t K,
                              uint32_t M, uint32_t row_offset, const uint32_t* rows,
                              uint32_t n_rows);
void orc_batch_matmul_q4k_rows(const uint8_t* W, const float* X, float* Y, uint32_t N,
                               uint32_t K, uint32_t M, uint32_t row_offset,
                               const uint32_t* rows, uint32_t n_rows);

/* batch_matmul_swiglu_q8 (llm.slang:1769-1911): Wg, Wu Q8_0 [N, K] (rows from
 * 0), all f32 (a = x, b = f32(d)*q), out = silu(g) * u, silu(g) = g/(1+exp(-g));
 * X f32 [M, K], Y f32 [M, N] (the _rows form: [n_rows, N]). */
void orc_batch_matmul_swiglu_q8(const uint8_t* Wg, const uint8_t* Wu, const float* X, float* Y, uint32_t N,
                                uint32_t K, uint32_t M);
void orc_batch_matmul_swiglu_q8_rows(const uint8_t* Wg, const uint8_t* Wu, const float* X, float* Y,
                                     uint32_t N, uint32_t K, uint32_t M, const uint32_t* rows,
                                     uint32_t n_rows);

/* flash_attention_v2 (flash_attn.slang:38-241): Q/K/V f32 [H,S,D] rounded to
 * fp16, BR=16 query rows, BC=32 key tiles, f32 online softmax, tree-reduced
 * tile sums; O f32 [S, H*D]. Restricted to heads [h0, h1) and query rows
 * [q0, q1) so large shapes can be sampled; rows outside are left untouched. */
void orc_flash_attention(const float* Q, const float* K, const float* V, float* O, uint32_t D,
                         uint32_t H, uint32_t S, float scale, uint32_t h0, uint32_t h1,
                         uint32_t q0, uint32_t q1);

/* Flux RoPE tables (flux_dit.c3:396-529 generalised to n_axes axes) and the
 * interleaved-pair rotation of mrope.slang:47-53 on [H,S,128] data. */
void orc_rope_tables(const uint32_t* pos /* [S, n_axes] */, uint32_t S, const uint32_t* axes_dims,
                     uint32_t n_axes, float theta, float* cos_out, float* sin_out);
void orc_rope_apply(float* x, uint32_t H, uint32_t S, const float* cos_t, const float* sin_t);

/* DiT block glue, one function per reference dispatch (zimage.slang,
 * diffusion.slang), f32, reference reduction order (256 strided partial sums,
 * then the shared-memory tree). */
void orc_batch_rmsnorm(const float* x, const float* w, float* out, uint32_t dim, uint32_t n_rows, float eps);
void orc_batch_layernorm(const float* x, float* out, uint32_t dim, uint32_t n_rows, float eps);
void orc_modulate(float* x, const float* scale, const float* shift /* NULL: scale_modulate */, uint32_t dim,
                  size_t n);
void orc_batch_head_norm(float* x, const float* w, uint32_t n_heads, uint32_t D, uint32_t seq_len, float eps);
void orc_transpose_heads(const float* in, float* out, uint32_t S, uint32_t H, uint32_t D);
void orc_gated_residual(float* residual, const float* gate, const float* input, uint32_t dim, size_t n,
                        int tanh_gate, float scale, float clip_thresh);
void orc_silu(float* x, size_t n);
void orc_gelu(float* x, size_t n);
void orc_timestep_embed(float* out, uint32_t dim, float t);
void orc_patchify(const float* in, float* out, uint32_t C, uint32_t H, uint32_t W, uint32_t ps);
void orc_unpatchify(const float* in, float* out, uint32_t C, uint32_t H, uint32_t W, uint32_t ps);

/* LoRA: the two-hop correction (hop 1 down-projection, hop 2 scaled
 * accumulate) and the load-time Q8_0 merge with requantization. */
void orc_lora_down(const float* A, const float* X, float* scratch, uint32_t rank, uint32_t in_dim,
                   uint32_t seq_len);
void orc_lora_up(const float* B, const float* scratch, float* out, uint32_t rank, uint32_t out_dim,
                 uint32_t seq_len, float scale, uint32_t row_offset, uint32_t weight_row_offset, uint32_t b_rows);
void orc_q8_lora_merge(uint8_t* base, const float* A, const float* B, uint32_t in_dim, uint32_t b_rows,
                       uint32_t dst_row_offset, uint32_t rank, float scale);

/* Number of OpenMP threads the oracle uses. */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif
