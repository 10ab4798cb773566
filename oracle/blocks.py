"""CPU restatement of the DiT block call sequences, built from the oracle's
per-dispatch functions (oracle.py / oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for llmr_amd.dit. Imported by tests/
and never by the product.

Every intermediate is an f32 buffer, as in the reference; the GEMMs and
attention apply their own operand rounding (batch_matmul_q8: fp16 x and the
RN_fp16(d*q) weight, llm.slang:1673-1703; batch_matmul_q4k: all f32,
llm.slang:2264-2365; flash_attention_v2: fp16 Q/K/V, flash_attn.slang:38-241).

  zimage_layer   dit_transformer_layer with adaLN (dependencies/zimage.c3l/
                 dit.c3:1372-1627): batch_rmsnorm, scale_modulate, 3 slot
                 GEMMs, batch_head_norm x2, transpose_heads x3, mrope x2,
                 flash_attention_v2, O-proj, batch_rmsnorm, gated_residual,
                 batch_rmsnorm, scale_modulate, batch_matmul_swiglu_q8, down
                 GEMM, batch_rmsnorm, gated_residual.
  flux_forward   FluxDiTModel.forward (dependencies/flux.c3l/flux_dit.c3:
                 1075-1210) with the choices of llmr_amd.dit.FluxDiT (per-block
                 modulation; the Flux.1-dev GELU MLP or the reference's own
                 SwiGLU MLP, cfg.mlp_act), each block the reference's dispatch
                 order (flux_dit.c3:746-1071).
"""
from __future__ import annotations

import math

import numpy as np

from . import oracle as orc

GGML_Q8_0, GGML_Q4_K = 8, 12


def _mm(W, wtype, X, N, row_offset=0):
    X = np.ascontiguousarray(X, np.float32)
    return orc.batch_matmul(W, wtype, X, N, X.shape[1], X.shape[0], row_offset)


def zimage_layer(w: dict, hidden: np.ndarray, n_heads: int, cos_t, sin_t, eps: float = 1e-5,
                 rows=None) -> np.ndarray:
    """w: numpy copies of llmr_amd.dit.ZImageLayerWeights fields (raw Q8_0
    blocks, f32 vectors). Returns the updated hidden (f32 [S, dim]); with
    `rows` only those rows' updates are computed (K and V of every row, the
    rest of the layer on the rows) and returned as [len(rows), dim]."""
    S, dim = hidden.shape
    ffn = w["w_gate"].size // (dim // 32 * 34)  # Q8_0 rows of dim/32 34-byte blocks
    h = np.array(hidden, np.float32, copy=True)
    scale_msa, gate_msa, scale_mlp, gate_mlp = (w["adaln"][i] for i in range(4))
    a = orc.modulate(orc.batch_rmsnorm(h, w["attn_norm1"], eps), scale_msa)
    k = _mm(w["wqkv"], GGML_Q8_0, a, dim, dim)
    v = _mm(w["wqkv"], GGML_Q8_0, a, dim, 2 * dim)
    if rows is None:
        q = _mm(w["wqkv"], GGML_Q8_0, a, dim, 0)
    else:
        rows = np.asarray(rows)
        q = np.zeros((S, dim), np.float32)
        q[rows] = _mm_rows(w["wqkv"], GGML_Q8_0, a, dim, 0, rows)
        h = h[rows]
    q = orc.batch_head_norm(q, w["q_norm"], n_heads, eps)
    k = orc.batch_head_norm(k, w["k_norm"], n_heads, eps)
    o = _attention_rows(q, k, v, n_heads, cos_t, sin_t, rows)
    t = _mm(w["wo"], GGML_Q8_0, o, dim)
    h = orc.gated_residual(h, gate_msa, orc.batch_rmsnorm(t, w["attn_norm2"], eps), True)
    a = orc.modulate(orc.batch_rmsnorm(h, w["ffn_norm1"], eps), scale_mlp)
    f = orc.batch_matmul_swiglu_q8(w["w_gate"], w["w_up"], a, ffn, dim, h.shape[0])
    t = _mm(w["w_down"], GGML_Q8_0, f, dim)
    return orc.gated_residual(h, gate_mlp, orc.batch_rmsnorm(t, w["ffn_norm2"], eps), True)


def _ln_mod(x, shift, scale, eps=1e-6):
    return orc.modulate(orc.batch_layernorm(x, eps), scale, shift)


def _row_ranges(rows, S):
    """Sorted query rows -> the 16-aligned [lo, hi) ranges covering them (the
    oracle attention computes whole 16-query blocks)."""
    if rows is None:
        return [(0, S)]
    out = []
    for b in sorted({int(r) // 16 for r in rows}):
        lo, hi = 16 * b, min(16 * b + 16, S)
        if out and out[-1][1] == lo:
            out[-1] = (out[-1][0], hi)
        else:
            out.append((lo, hi))
    return out


def _attention_rows(q_rows, k_rows, v_rows, n_heads, cos_t, sin_t, rows):
    """transpose_heads x3, mrope on Q and K, flash_attention_v2: the attention
    output [len(rows), H*128] of the query rows `rows` (all rows, [S, H*128],
    when None); q_rows [S, H*128] holds Q for at least those rows, K/V all."""
    S = k_rows.shape[0]
    q = orc.rope_apply(orc.transpose_heads(q_rows, n_heads), cos_t, sin_t)
    k = orc.rope_apply(orc.transpose_heads(k_rows, n_heads), cos_t, sin_t)
    v = orc.transpose_heads(v_rows, n_heads)
    scale = 1.0 / math.sqrt(128.0)
    if rows is None:
        return orc.flash_attention(q, k, v, scale)
    o = np.full((S, q_rows.shape[1]), np.nan, np.float32)
    for lo, hi in _row_ranges(rows, S):
        o[lo:hi] = orc.flash_attention(q, k, v, scale, qrange=(lo, hi))[lo:hi]
    return o[np.asarray(rows)]


def _mm_rows(W, wtype, X, N, row_offset, rows):
    """GEMM of the rows `rows` of X (all rows when None)."""
    X = np.ascontiguousarray(X, np.float32)
    if rows is None:
        return orc.batch_matmul(W, wtype, X, N, X.shape[1], X.shape[0], row_offset)
    return orc.batch_matmul(W, wtype, X, N, X.shape[1], X.shape[0], row_offset, rows=np.asarray(rows))


def _mlp_in(W, a, m, mlp_act, row0=0, rows=None):
    """The MLP in-projection of a block and its activation: GELU of m rows
    from row0 (the Flux.1-dev form), or silu(gate) * up of the m gate rows
    from row0 and the m up rows after them (the reference's Flux.2 form:
    flux_matmul of the gate and up slots, then silu and elemwise_mul in f32,
    flux_dit.c3:917-931, 1013-1018, 1049-1055)."""
    if mlp_act == "gelu":
        return orc.gelu(_mm_rows(W, GGML_Q4_K, a, m, row0, rows))
    g = _mm_rows(W, GGML_Q4_K, a, m, row0, rows)
    u = _mm_rows(W, GGML_Q4_K, a, m, row0 + m, rows)
    return orc.silu(g) * u


def flux_double_block(w: dict, txt_h: np.ndarray, img: np.ndarray, mt: np.ndarray, mi: np.ndarray, n_heads: int,
                      cos_t, sin_t, rows=None, mlp_act: str = "gelu"):
    """flux_dual_stream_block (flux_dit.c3:746-971). mlp_act "gelu": the
    Flux.1-dev GELU MLP ([m, d] in-projection); "swiglu": the reference's own
    SwiGLU MLP ([2 m, d]: gate rows, then up rows). txt_h [n_txt, d] / img
    [n_img, d]: the two residual streams; mt / mi [6, d]: (shift1, scale1,
    gate1, shift2, scale2, gate2) of each stream. Returns the updated (txt_h,
    img); with `rows` (joint row indices, text rows first) only those rows'
    updates are computed and returned as one [len(rows), d] array in joint
    order."""
    d = txt_h.shape[1]
    nt, ni = txt_h.shape[0], img.shape[0]
    m = w["img_mlp0"].size // (d // 256 * 144) // (2 if mlp_act == "swiglu" else 1)
    eps_hn = 1e-6
    a_i = _ln_mod(img, mi[0], mi[1])
    a_t = _ln_mod(txt_h, mt[0], mt[1])
    # K, V of every joint row; Q of the rows asked for
    ki, vi = (_mm(w["img_qkv"], GGML_Q4_K, a_i, d, r * d) for r in (1, 2))
    kt, vt = (_mm(w["txt_qkv"], GGML_Q4_K, a_t, d, r * d) for r in (1, 2))
    if rows is None:
        qt, qi = _mm(w["txt_qkv"], GGML_Q4_K, a_t, d, 0), _mm(w["img_qkv"], GGML_Q4_K, a_i, d, 0)
        q = np.concatenate([qt, qi])
    else:
        rows = np.asarray(rows)
        q = np.zeros((nt + ni, d), np.float32)
        rt, ri = rows[rows < nt], rows[rows >= nt] - nt
        if rt.size:
            q[rt] = _mm_rows(w["txt_qkv"], GGML_Q4_K, a_t, d, 0, rt)
        if ri.size:
            q[ri + nt] = _mm_rows(w["img_qkv"], GGML_Q4_K, a_i, d, 0, ri)
    q = np.concatenate([orc.batch_head_norm(q[:nt], w["txt_q_norm"], n_heads, eps_hn),
                        orc.batch_head_norm(q[nt:], w["img_q_norm"], n_heads, eps_hn)])
    k = np.concatenate([orc.batch_head_norm(kt, w["txt_k_norm"], n_heads, eps_hn),
                        orc.batch_head_norm(ki, w["img_k_norm"], n_heads, eps_hn)])
    v = np.concatenate([vt, vi])
    o = _attention_rows(q, k, v, n_heads, cos_t, sin_t, rows)

    def stream(h, mod, wp, w0, w2, o_s):
        """Attention projection + gated residual, then the MLP half."""
        h = orc.gated_residual(h, mod[2], _mm(wp, GGML_Q4_K, o_s, d), False)
        a = _ln_mod(h, mod[3], mod[4])
        return orc.gated_residual(h, mod[5], _mm(w2, GGML_Q4_K, _mlp_in(w0, a, m, mlp_act), d), False)

    if rows is None:
        txt_h = stream(txt_h, mt, w["txt_proj"], w["txt_mlp0"], w["txt_mlp2"], o[:nt])
        img = stream(img, mi, w["img_proj"], w["img_mlp0"], w["img_mlp2"], o[nt:])
        return txt_h, img
    out = np.empty((rows.size, d), np.float32)
    sel_t, sel_i = rows < nt, rows >= nt
    if sel_t.any():
        out[sel_t] = stream(txt_h[rows[sel_t]], mt, w["txt_proj"], w["txt_mlp0"], w["txt_mlp2"], o[sel_t])
    if sel_i.any():
        out[sel_i] = stream(img[rows[sel_i] - nt], mi, w["img_proj"], w["img_mlp0"], w["img_mlp2"], o[sel_i])
    return out


def flux_single_block(w: dict, h: np.ndarray, ms: np.ndarray, n_heads: int, cos_t, sin_t, rows=None,
                      mlp_act: str = "gelu"):
    """flux_single_stream_block (flux_dit.c3:975-1071). mlp_act "gelu": the
    Flux.1-dev GELU MLP half of linear1 ([3 d + m, d]); "swiglu": the
    reference's own form, linear1 [3 d + 2 m, d] whose last 2 m rows are a
    SwiGLU gate and up (flux_dit.c3:1013-1018, 1049-1055). h [S, d] joint
    stream (text rows first); ms [3, d] (shift, scale, gate). Returns the
    updated h, or with `rows` the updated rows [len(rows), d]."""
    S, d = h.shape
    m = (w["linear1"].size // (d // 256 * 144) - 3 * d) // (2 if mlp_act == "swiglu" else 1)
    eps_hn = 1e-6
    a = _ln_mod(h, ms[0], ms[1])
    k, v = (_mm(w["linear1"], GGML_Q4_K, a, d, r * d) for r in (1, 2))
    if rows is None:
        q = _mm(w["linear1"], GGML_Q4_K, a, d, 0)
        mlp = _mlp_in(w["linear1"], a, m, mlp_act, 3 * d)
        h_r = h
    else:
        rows = np.asarray(rows)
        q = np.zeros((S, d), np.float32)
        q[rows] = _mm_rows(w["linear1"], GGML_Q4_K, a, d, 0, rows)
        mlp = _mlp_in(w["linear1"], a, m, mlp_act, 3 * d, rows)
        h_r = h[rows]
    q = orc.batch_head_norm(q, w["q_norm"], n_heads, eps_hn)
    k = orc.batch_head_norm(k, w["k_norm"], n_heads, eps_hn)
    o = _attention_rows(q, k, v, n_heads, cos_t, sin_t, rows)
    cat = np.concatenate([o, mlp], axis=1)
    return orc.gated_residual(h_r, ms[2], _mm(w["linear2"], GGML_Q4_K, cat, d), False)


def flux_forward(cfg, glob: dict, doubles: list, singles: list, latent: np.ndarray, txt: np.ndarray,
                 sigma: float, cos_t, sin_t) -> np.ndarray:
    """cfg: llmr_amd.dit.FluxConfig; weights: dicts of numpy copies of the
    FluxGlobalWeights / FluxDoubleWeights / FluxSingleWeights fields. Returns
    the velocity f32 [C, H, W]."""
    d, H, nt = cfg.dim, cfg.n_heads, cfg.n_txt
    patches = orc.patchify(latent, cfg.patch)
    img = _mm(glob["img_in"], GGML_Q8_0, patches, d)
    txt_h = _mm(glob["txt_in"], GGML_Q4_K, txt, d)
    temb = orc.timestep_embed(cfg.t_emb_dim, sigma * 1000.0)[None, :]
    vec = _mm(glob["time_in1"], GGML_Q4_K, orc.silu(_mm(glob["time_in0"], GGML_Q4_K, temb, d)), d)
    vec = orc.silu(vec)
    mod = lambda W, n: _mm(W, GGML_Q4_K, vec, n * d).reshape(n, d)  # noqa: E731
    act = getattr(cfg, "mlp_act", "gelu")
    for w in doubles:
        txt_h, img = flux_double_block(w, txt_h, img, mod(w["txt_mod"], 6), mod(w["img_mod"], 6), H, cos_t, sin_t,
                                       mlp_act=act)
    h = np.concatenate([txt_h, img])
    for w in singles:
        h = flux_single_block(w, h, mod(w["mod"], 3), H, cos_t, sin_t, mlp_act=act)
    fm = mod(glob["final_mod"], 2)
    a = _ln_mod(h[nt:], fm[0], fm[1])
    vel = _mm(glob["final_linear"], GGML_Q4_K, a, cfg.patch_dim)
    return orc.unpatchify(vel, cfg.latent_ch, cfg.latent_h, cfg.latent_w, cfg.patch)
