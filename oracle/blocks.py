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
                 1075-1210) with the Flux.1-dev choices of llmr_amd.dit.FluxDiT
                 (GELU MLP, per-block modulation), each block the reference's
                 dispatch order (flux_dit.c3:746-1071).
"""
from __future__ import annotations

import math

import numpy as np

from . import oracle as orc

GGML_Q8_0, GGML_Q4_K = 8, 12


def _mm(W, wtype, X, N, row_offset=0):
    X = np.ascontiguousarray(X, np.float32)
    return orc.batch_matmul(W, wtype, X, N, X.shape[1], X.shape[0], row_offset)


def _attention_from_rows(q_rows, k_rows, v_rows, n_heads, cos_t, sin_t):
    """transpose_heads x3, mrope on Q and K, flash_attention_v2 -> O [S, H*128]."""
    q = orc.rope_apply(orc.transpose_heads(q_rows, n_heads), cos_t, sin_t)
    k = orc.rope_apply(orc.transpose_heads(k_rows, n_heads), cos_t, sin_t)
    v = orc.transpose_heads(v_rows, n_heads)
    return orc.flash_attention(q, k, v, 1.0 / math.sqrt(128.0))


def zimage_layer(w: dict, hidden: np.ndarray, n_heads: int, cos_t, sin_t, eps: float = 1e-5) -> np.ndarray:
    """w: numpy copies of llmr_amd.dit.ZImageLayerWeights fields (raw Q8_0
    blocks, f32 vectors). Returns the updated hidden (f32 [S, dim])."""
    S, dim = hidden.shape
    ffn = w["w_gate"].size // (dim // 32 * 34)  # Q8_0 rows of dim/32 34-byte blocks
    h = np.array(hidden, np.float32, copy=True)
    scale_msa, gate_msa, scale_mlp, gate_mlp = (w["adaln"][i] for i in range(4))
    a = orc.modulate(orc.batch_rmsnorm(h, w["attn_norm1"], eps), scale_msa)
    q = _mm(w["wqkv"], GGML_Q8_0, a, dim, 0)
    k = _mm(w["wqkv"], GGML_Q8_0, a, dim, dim)
    v = _mm(w["wqkv"], GGML_Q8_0, a, dim, 2 * dim)
    q = orc.batch_head_norm(q, w["q_norm"], n_heads, eps)
    k = orc.batch_head_norm(k, w["k_norm"], n_heads, eps)
    o = _attention_from_rows(q, k, v, n_heads, cos_t, sin_t)
    t = _mm(w["wo"], GGML_Q8_0, o, dim)
    h = orc.gated_residual(h, gate_msa, orc.batch_rmsnorm(t, w["attn_norm2"], eps), True)
    a = orc.modulate(orc.batch_rmsnorm(h, w["ffn_norm1"], eps), scale_mlp)
    f = orc.batch_matmul_swiglu_q8(w["w_gate"], w["w_up"], a, ffn, dim, S)
    t = _mm(w["w_down"], GGML_Q8_0, f, dim)
    return orc.gated_residual(h, gate_mlp, orc.batch_rmsnorm(t, w["ffn_norm2"], eps), True)


def _ln_mod(x, shift, scale, eps=1e-6):
    return orc.modulate(orc.batch_layernorm(x, eps), scale, shift)


def flux_forward(cfg, glob: dict, doubles: list, singles: list, latent: np.ndarray, txt: np.ndarray,
                 sigma: float, cos_t, sin_t) -> np.ndarray:
    """cfg: llmr_amd.dit.FluxConfig; weights: dicts of numpy copies of the
    FluxGlobalWeights / FluxDoubleWeights / FluxSingleWeights fields. Returns
    the velocity f32 [C, H, W]."""
    d, m, H, nt = cfg.dim, cfg.mlp, cfg.n_heads, cfg.n_txt
    patches = orc.patchify(latent, cfg.patch)
    img = _mm(glob["img_in"], GGML_Q8_0, patches, d)
    txt_h = _mm(glob["txt_in"], GGML_Q4_K, txt, d)
    temb = orc.timestep_embed(cfg.t_emb_dim, sigma * 1000.0)[None, :]
    vec = _mm(glob["time_in1"], GGML_Q4_K, orc.silu(_mm(glob["time_in0"], GGML_Q4_K, temb, d)), d)
    vec = orc.silu(vec)
    mod = lambda W, n: _mm(W, GGML_Q4_K, vec, n * d).reshape(n, d)  # noqa: E731
    eps_hn = 1e-6
    for w in doubles:
        mi, mt = mod(w["img_mod"], 6), mod(w["txt_mod"], 6)
        a_i = _ln_mod(img, mi[0], mi[1])
        a_t = _ln_mod(txt_h, mt[0], mt[1])
        qi, ki, vi = (_mm(w["img_qkv"], GGML_Q4_K, a_i, d, r * d) for r in range(3))
        qt, kt, vt = (_mm(w["txt_qkv"], GGML_Q4_K, a_t, d, r * d) for r in range(3))
        q = np.concatenate([orc.batch_head_norm(qt, w["txt_q_norm"], H, eps_hn),
                            orc.batch_head_norm(qi, w["img_q_norm"], H, eps_hn)])
        k = np.concatenate([orc.batch_head_norm(kt, w["txt_k_norm"], H, eps_hn),
                            orc.batch_head_norm(ki, w["img_k_norm"], H, eps_hn)])
        v = np.concatenate([vt, vi])
        o = _attention_from_rows(q, k, v, H, cos_t, sin_t)
        txt_o = _mm(w["txt_proj"], GGML_Q4_K, o[:nt], d)
        img_o = _mm(w["img_proj"], GGML_Q4_K, o[nt:], d)
        img = orc.gated_residual(img, mi[2], img_o, False)
        txt_h = orc.gated_residual(txt_h, mt[2], txt_o, False)
        a_i = _ln_mod(img, mi[3], mi[4])
        img = orc.gated_residual(img, mi[5], _mm(w["img_mlp2"], GGML_Q4_K,
                                                 orc.gelu(_mm(w["img_mlp0"], GGML_Q4_K, a_i, m)), d), False)
        a_t = _ln_mod(txt_h, mt[3], mt[4])
        txt_h = orc.gated_residual(txt_h, mt[5], _mm(w["txt_mlp2"], GGML_Q4_K,
                                                     orc.gelu(_mm(w["txt_mlp0"], GGML_Q4_K, a_t, m)), d), False)
    h = np.concatenate([txt_h, img])
    for w in singles:
        ms = mod(w["mod"], 3)
        a = _ln_mod(h, ms[0], ms[1])
        q, k, v = (_mm(w["linear1"], GGML_Q4_K, a, d, r * d) for r in range(3))
        mlp = orc.gelu(_mm(w["linear1"], GGML_Q4_K, a, m, 3 * d))
        q = orc.batch_head_norm(q, w["q_norm"], H, eps_hn)
        k = orc.batch_head_norm(k, w["k_norm"], H, eps_hn)
        o = _attention_from_rows(q, k, v, H, cos_t, sin_t)
        cat = np.concatenate([o, mlp], axis=1)
        h = orc.gated_residual(h, ms[2], _mm(w["linear2"], GGML_Q4_K, cat, d), False)
    fm = mod(glob["final_mod"], 2)
    a = _ln_mod(h[nt:], fm[0], fm[1])
    vel = _mm(glob["final_linear"], GGML_Q4_K, a, cfg.patch_dim)
    return orc.unpatchify(vel, cfg.latent_ch, cfg.latent_h, cfg.latent_w, cfg.patch)
