"""The oracle's block compositions (oracle/blocks.py) pinned against float64
restatements of the reference's block definitions and against closed forms.

The per-dispatch oracle functions are pinned one by one elsewhere; what these
tests pin is the composition: which adaLN chunk feeds which norm, which
weight slot is Q, K or V, the post-norms, tanh against linear gates, text
rows before image rows, RoPE on Q and K only. The float64 restatement here
is written from the reference's block functions (dependencies/zimage.c3l/
dit.c3:1372-1627, dependencies/flux.c3l/flux_dit.c3:746-1210) with dense
float64 matrices (the f32 dequantized weights, which are exact), textbook
two-pass softmax and no operand rounding, so it shares no arithmetic with
the oracle beyond the dequantized weight values and the RoPE tables.

Each plausible composition mistake is planted in the float64 restatement
(`mistake=`); the test shows the planted version is far from the oracle
(more than 10x the tolerance), so an oracle carrying that mistake could not
pass the tolerance against the correct restatement.
"""
import math

import numpy as np
import pytest

from conftest import rel_l2

Q8, Q4K = 8, 12


# ---------------------------------------------------------------------------
# float64 restatement of the reference's block functions
# ---------------------------------------------------------------------------

def _deq(orc, blocks, wtype, rows, cols):
    """The f32 dequantized weight (exact: tensor.c3:319-361) as float64 [rows, cols]."""
    f = orc.dequant_q8_0 if wtype == Q8 else orc.dequant_q4k
    return f(np.asarray(blocks, np.uint8).reshape(-1)).astype(np.float64).reshape(rows, cols)


def _rms(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def _ln(x, eps):
    mu = x.mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)


def _head_norm(x, w, H, eps):
    S = x.shape[0]
    return _rms(x.reshape(S, H, 128), w, eps).reshape(S, H * 128)


def _rope(x, cos_t, sin_t):
    """Interleaved pairs (2j, 2j+1) of each head row (mrope.slang:47-53); x [S, H*128]."""
    S = x.shape[0]
    y = x.reshape(S, -1, 64, 2).copy()
    c, s = cos_t[:, None, :], sin_t[:, None, :]
    x0, x1 = y[..., 0].copy(), y[..., 1].copy()
    y[..., 0] = x0 * c - x1 * s
    y[..., 1] = x0 * s + x1 * c
    return y.reshape(S, -1)


def _attention(q, k, v, H):
    """Textbook softmax(q k^T / sqrt(128)) v per head; [S, H*128] -> [S, H*128]."""
    S = q.shape[0]
    o = np.empty((S, H * 128))
    for h in range(H):
        sl = slice(128 * h, 128 * h + 128)
        sc = q[:, sl] @ k[:, sl].T / math.sqrt(128.0)
        p = np.exp(sc - sc.max(1, keepdims=True))
        o[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    return o


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def zimage_f64(orc, w, h, H, cos_t, sin_t, eps=1e-5, mistake=None):
    """dit_transformer_layer with adaLN (dit.c3:1372-1627) in float64.
    adaln chunks: scale_msa, gate_msa, scale_mlp, gate_mlp (dit.c3:1403-1416,
    1517-1533)."""
    S, d = h.shape
    ffn = np.asarray(w["w_gate"]).size // (d // 32 * 34)
    W = lambda key, n, k: _deq(orc, w[key], Q8, n, k)  # noqa: E731
    wqkv = W("wqkv", 3 * d, d)
    ad = np.asarray(w["adaln"], np.float64)
    sc_msa, g_msa, sc_mlp, g_mlp = ad[0], ad[1], ad[2], ad[3]
    if mistake == "swap_scales":
        sc_msa, sc_mlp = sc_mlp, sc_msa
    if mistake == "swap_gates":
        g_msa, g_mlp = g_mlp, g_msa
    gate = (lambda g: g) if mistake == "linear_gate" else np.tanh
    n = {k: np.asarray(w[k], np.float64) for k in ("attn_norm1", "attn_norm2", "ffn_norm1", "ffn_norm2",
                                                   "q_norm", "k_norm")}
    h = np.asarray(h, np.float64)
    a = _rms(h, n["attn_norm1"], eps) * (1.0 + sc_msa)
    q, k, v = (a @ wqkv[r * d:(r + 1) * d].T for r in range(3))
    if mistake == "kv_slots":
        k, v = v, k
    q = _head_norm(q, n["q_norm"], H, eps)
    k = _head_norm(k, n["k_norm" if mistake != "q_norm_for_k" else "q_norm"], H, eps)
    if mistake != "no_rope":
        q, k = _rope(q, cos_t, sin_t), _rope(k, cos_t, sin_t)
    o = _attention(q, k, v, H)
    t = o @ W("wo", d, d).T
    post = (lambda x, nw: x) if mistake == "no_postnorm" else (lambda x, nw: _rms(x, nw, eps))
    h = h + gate(g_msa) * post(t, n["attn_norm2"])
    a = _rms(h, n["ffn_norm1"], eps) * (1.0 + sc_mlp)
    f = _silu(a @ W("w_gate", ffn, d).T) * (a @ W("w_up", ffn, d).T)
    t = f @ W("w_down", d, ffn).T
    return h + gate(g_mlp) * post(t, n["ffn_norm2"])


def _patchify(x, p):
    C, Hh, Ww = x.shape
    return x.reshape(C, Hh // p, p, Ww // p, p).transpose(1, 3, 2, 4, 0).reshape((Hh // p) * (Ww // p), p * p * C)


def _unpatchify(y, C, Hh, Ww, p):
    return y.reshape(Hh // p, Ww // p, p, p, C).transpose(4, 0, 2, 1, 3).reshape(C, Hh, Ww)


def _timestep(dim, t):
    half = dim // 2
    freq = np.exp(-math.log(10000.0) * np.arange(half) / half)
    return np.concatenate([np.cos(t * freq), np.sin(t * freq)])


def flux_f64(orc, cfg, glob, doubles, singles, latent, txt, sigma, cos_t, sin_t, mistake=None):
    """FluxDiTModel.forward (flux_dit.c3:1075-1210) in float64 with
    per-block modulation and cfg.mlp_act's MLP: the Flux.1-dev GELU, or the
    reference's SwiGLU (silu of the gate rows times the up rows after them,
    flux_dit.c3:917-931, 1013-1018, 1049-1055). Chunks per stream of a
    double block: shift1, scale1, gate1, shift2, scale2, gate2
    (flux_dit.c3:764-765,889,905-906,936); single block: shift, scale, gate
    (:988-989,1064); final layer: shift, scale (:1183-1185)."""
    d, m, H, nt = cfg.dim, cfg.mlp, cfg.n_heads, cfg.n_txt
    swiglu = cfg.mlp_act == "swiglu"

    def mlp_in(a, W):
        """a @ W.T of the MLP in-projection rows W, activated."""
        if not swiglu:
            return _gelu(a @ W.T)
        g, u = a @ W[:m].T, a @ W[m:].T
        if mistake == "swiglu_halves":
            g, u = u, g
        if mistake == "swiglu_gelu":
            return _gelu(g) * u
        if mistake == "swiglu_no_gate":
            return u
        return _silu(g) * u
    G = lambda blocks, wt, n, k: _deq(orc, blocks, wt, n, k)  # noqa: E731
    eps = 1e-6
    img = _patchify(np.asarray(latent, np.float64), cfg.patch) @ G(glob["img_in"], Q8, d, cfg.patch_dim).T
    txt_h = np.asarray(txt, np.float64) @ G(glob["txt_in"], Q4K, d, cfg.text_dim).T
    vec = _silu(_timestep(cfg.t_emb_dim, sigma * 1000.0) @ G(glob["time_in0"], Q4K, d, cfg.t_emb_dim).T)
    vec = vec @ G(glob["time_in1"], Q4K, d, d).T
    if mistake != "no_vec_silu":
        vec = _silu(vec)

    def mod(blocks, n):
        c = (vec @ G(blocks, Q4K, n * d, d).T).reshape(n, d)
        if mistake == "shift_scale":
            c[[0, 1]] = c[[1, 0]]
        return c

    def ln_mod(x, shift, scale):
        return _ln(x, eps) * (1.0 + scale) + shift

    cos64, sin64 = np.asarray(cos_t, np.float64), np.asarray(sin_t, np.float64)
    for w in doubles:
        mi, mt = mod(w["img_mod"], 6), mod(w["txt_mod"], 6)
        if mistake == "stream_mods":
            mi, mt = mt, mi
        a_i, a_t = ln_mod(img, mi[0], mi[1]), ln_mod(txt_h, mt[0], mt[1])
        wi, wt = G(w["img_qkv"], Q4K, 3 * d, d), G(w["txt_qkv"], Q4K, 3 * d, d)
        qi, ki, vi = (a_i @ wi[r * d:(r + 1) * d].T for r in range(3))
        qt, kt, vt = (a_t @ wt[r * d:(r + 1) * d].T for r in range(3))
        nq = lambda x, key: _head_norm(x, np.asarray(w[key], np.float64), H, eps)  # noqa: E731
        if mistake == "no_head_norm":
            nq = lambda x, key: x  # noqa: E731
        q = np.concatenate([nq(qt, "txt_q_norm"), nq(qi, "img_q_norm")])
        k = np.concatenate([nq(kt, "txt_k_norm"), nq(ki, "img_k_norm")])
        v = np.concatenate([vt, vi])
        if mistake == "image_first":
            q, k, v = (np.concatenate([x[nt:], x[:nt]]) for x in (q, k, v))
        o = _attention(_rope(q, cos64, sin64), _rope(k, cos64, sin64), v, H)
        if mistake == "image_first":
            o = np.concatenate([o[-nt:], o[:-nt]])
        g1, g2 = (2, 5) if mistake != "gate_chunks" else (5, 2)
        txt_h = txt_h + mt[g1] * (o[:nt] @ G(w["txt_proj"], Q4K, d, d).T)
        img = img + mi[g1] * (o[nt:] @ G(w["img_proj"], Q4K, d, d).T)
        a_i, a_t = ln_mod(img, mi[3], mi[4]), ln_mod(txt_h, mt[3], mt[4])
        mi_rows = cfg.mlp_in
        img = img + mi[g2] * (mlp_in(a_i, G(w["img_mlp0"], Q4K, mi_rows, d)) @ G(w["img_mlp2"], Q4K, d, m).T)
        txt_h = txt_h + mt[g2] * (mlp_in(a_t, G(w["txt_mlp0"], Q4K, mi_rows, d)) @ G(w["txt_mlp2"], Q4K, d, m).T)
    h = np.concatenate([txt_h, img])
    for w in singles:
        ms = mod(w["mod"], 3)
        a = ln_mod(h, ms[0], ms[1])
        l1 = G(w["linear1"], Q4K, 3 * d + cfg.mlp_in, d)
        q, k, v = (a @ l1[r * d:(r + 1) * d].T for r in range(3))
        mlp = mlp_in(a, l1[3 * d:])
        q = _head_norm(q, np.asarray(w["q_norm"], np.float64), H, eps)
        k = _head_norm(k, np.asarray(w["k_norm"], np.float64), H, eps)
        o = _attention(_rope(q, cos64, sin64), _rope(k, cos64, sin64), v, H)
        cat = np.concatenate([o, mlp], 1) if mistake != "cat_order" else np.concatenate([mlp, o], 1)
        h = h + ms[2] * (cat @ G(w["linear2"], Q4K, d, d + m).T)
    fm = (vec @ G(glob["final_mod"], Q4K, 2 * d, d).T).reshape(2, d)
    shift, scale = (fm[0], fm[1]) if mistake != "final_shift_scale" else (fm[1], fm[0])
    a = ln_mod(h[nt:], shift, scale)
    vel = a @ G(glob["final_linear"], Q4K, cfg.patch_dim, d).T
    return _unpatchify(vel, cfg.latent_ch, cfg.latent_h, cfg.latent_w, cfg.patch)


# ---------------------------------------------------------------------------
# weights on the host
# ---------------------------------------------------------------------------

def _zimage_weights(r, dim, ffn):
    from llmr_amd import gguf

    def q8(n, k):
        return gguf.quantize((0.05 * r.standard_normal((n, k))).astype(np.float32), gguf.GGML_Q8_0)

    def vec(n):
        return (1.0 + 0.1 * r.standard_normal(n)).astype(np.float32)
    return dict(wqkv=q8(3 * dim, dim), wo=q8(dim, dim), w_gate=q8(ffn, dim), w_up=q8(ffn, dim),
                w_down=q8(dim, ffn), attn_norm1=vec(dim), attn_norm2=vec(dim), ffn_norm1=vec(dim),
                ffn_norm2=vec(dim), q_norm=vec(128), k_norm=vec(128),
                adaln=(0.8 * r.standard_normal((4, dim))).astype(np.float32))


def _zimage_rope(S, grid=6):
    from oracle import oracle as orc
    pos = np.zeros((S, 3), np.uint32)
    pos[:, 0] = np.arange(S) // (grid * grid)
    pos[:, 1] = (np.arange(S) // grid) % grid
    pos[:, 2] = np.arange(S) % grid
    return orc.rope_tables(pos, (32, 48, 48), 256.0)


ZIMAGE_MISTAKES = ["swap_scales", "swap_gates", "linear_gate", "kv_slots", "q_norm_for_k", "no_rope",
                   "no_postnorm"]


@pytest.fixture(scope="module")
def zimage_case(orc):
    r = np.random.default_rng(11)
    dim, H, ffn, S = 256, 2, 512, 72
    w = _zimage_weights(r, dim, ffn)
    h = r.standard_normal((S, dim)).astype(np.float32)
    cos_t, sin_t = _zimage_rope(S)
    return w, h, H, cos_t, sin_t


ZIMAGE_TOL = 2e-3  # measured 5.6e-4: fp16 GEMM operands and fp16 Q/K/V in the oracle; float64 here


def test_zimage_layer_vs_float64(orc, zimage_case):
    from oracle import blocks
    w, h, H, cos_t, sin_t = zimage_case
    got = blocks.zimage_layer(w, h, H, cos_t, sin_t)
    ref = zimage_f64(orc, w, h, H, cos_t, sin_t)
    err = rel_l2(got - h, ref - h)
    print(f"zimage layer update: rel L2 {err:.2e}")
    assert err < ZIMAGE_TOL


@pytest.mark.parametrize("mistake", ZIMAGE_MISTAKES)
def test_zimage_layer_catches_planted_mistake(orc, zimage_case, mistake):
    from oracle import blocks
    w, h, H, cos_t, sin_t = zimage_case
    got = blocks.zimage_layer(w, h, H, cos_t, sin_t)
    bad = zimage_f64(orc, w, h, H, cos_t, sin_t, mistake=mistake)
    err = rel_l2(got - h, bad - h)
    print(f"{mistake}: rel L2 {err:.2e}")
    assert err > 10 * ZIMAGE_TOL


def test_zimage_layer_zero_qk_is_mean_of_v(orc):
    """Q and K weight slots zero: head norm and RoPE keep them zero, every score
    is 0 and attention is the uniform mean of V over the keys, the same for
    every query. With gate_mlp = 0 the layer adds one row vector to every row:
    tanh(gate_msa) * rmsnorm(mean_V . Wo^T) * attn_norm2."""
    from llmr_amd import gguf
    from oracle import blocks
    r = np.random.default_rng(12)
    dim, H, ffn, S = 256, 2, 512, 48
    w = _zimage_weights(r, dim, ffn)
    row = dim // 32 * 34
    w["wqkv"] = w["wqkv"].copy()
    w["wqkv"][:2 * dim * row] = 0  # Q8_0 blocks with d = 0 dequantize to 0
    w["adaln"] = w["adaln"].copy()
    w["adaln"][3] = 0.0
    h = r.standard_normal((S, dim)).astype(np.float32)
    cos_t, sin_t = _zimage_rope(S)
    got = blocks.zimage_layer(w, h, H, cos_t, sin_t) - h.astype(np.float64)
    a = _rms(h.astype(np.float64), w["attn_norm1"], 1e-5) * (1.0 + w["adaln"][0].astype(np.float64))
    wv = _deq(orc, w["wqkv"], gguf.GGML_Q8_0, 3 * dim, dim)[2 * dim:]
    mean_v = (a @ wv.T).mean(0)
    t = mean_v @ _deq(orc, w["wo"], gguf.GGML_Q8_0, dim, dim).T
    u = np.tanh(w["adaln"][1].astype(np.float64)) * _rms(t, w["attn_norm2"], 1e-5)
    err = max(rel_l2(got[i], u) for i in range(S))
    print(f"zero-QK update vs closed form: max row rel L2 {err:.2e}")
    assert err < 3e-3
    # and every row's update is the same vector (to the rounding of the f32 add)
    assert np.abs(got - got[0]).max() < 1e-5 * (1 + np.abs(h).max())


# ---------------------------------------------------------------------------
# Flux forward
# ---------------------------------------------------------------------------

def _flux_cfg(mlp_act="gelu"):
    from llmr_amd import dit
    return dit.FluxConfig(dim=256, n_heads=2, mlp=512, n_double=2, n_single=2, text_dim=256, n_txt=24,
                          latent_ch=16, latent_h=12, latent_w=12, patch=2, mlp_act=mlp_act)


def _flux_weights(r, cfg, zero_gates=False):
    """Host-quantized weights shaped as llmr_amd.dit.flux_weights (as numpy
    dicts). Modulation weights have std 0.1 so that shifts, scales and gates
    are O(1) and distinct; with zero_gates every gate chunk's rows are zero
    blocks."""
    from llmr_amd import gguf
    d, m, mi = cfg.dim, cfg.mlp, cfg.mlp_in

    def q(n, k, std=0.05, wt=gguf.GGML_Q4_K):
        return gguf.quantize((std * r.standard_normal((n, k))).astype(np.float32), wt)

    def mod(n_chunks, gates):
        blk = q(n_chunks * d, d, 0.1)
        if zero_gates:
            row = d // 256 * 144
            for c in gates:
                blk[c * d * row:(c + 1) * d * row] = 0
        return blk

    def norm():
        return (1.0 + 0.1 * r.standard_normal(128)).astype(np.float32)
    doubles = [dict(img_mod=mod(6, (2, 5)), txt_mod=mod(6, (2, 5)), img_qkv=q(3 * d, d), txt_qkv=q(3 * d, d),
                    img_proj=q(d, d), txt_proj=q(d, d), img_mlp0=q(mi, d), txt_mlp0=q(mi, d), img_mlp2=q(d, m),
                    txt_mlp2=q(d, m), img_q_norm=norm(), img_k_norm=norm(), txt_q_norm=norm(),
                    txt_k_norm=norm()) for _ in range(cfg.n_double)]
    singles = [dict(mod=mod(3, (2,)), linear1=q(3 * d + mi, d), linear2=q(d, d + m), q_norm=norm(), k_norm=norm())
               for _ in range(cfg.n_single)]
    glob = dict(img_in=q(d, cfg.patch_dim, 0.1, gguf.GGML_Q8_0), txt_in=q(d, cfg.text_dim, 0.1),
                time_in0=q(d, cfg.t_emb_dim, 0.1), time_in1=q(d, d, 0.1), final_mod=q(2 * d, d, 0.1),
                final_linear=q(cfg.patch_dim, d, 0.1))
    return glob, doubles, singles


def _flux_inputs(r, cfg):
    from llmr_amd import dit
    lat = r.standard_normal((cfg.latent_ch, cfg.latent_h, cfg.latent_w)).astype(np.float32)
    txt = r.standard_normal((cfg.n_txt, cfg.text_dim)).astype(np.float32)
    cos_t, sin_t = (t.numpy() for t in dit.flux_rope(cfg, device="cpu"))
    return lat, txt, cos_t, sin_t


FLUX_TOL = 1e-3  # measured 1.4e-4: Q8_0 img_in with fp16 operands and fp16 Q/K/V in the oracle; float64 here
FLUX_MISTAKES = ["shift_scale", "gate_chunks", "stream_mods", "image_first", "no_head_norm", "no_vec_silu",
                 "cat_order", "final_shift_scale"]


@pytest.fixture(scope="module")
def flux_case(orc):
    from oracle import blocks
    cfg = _flux_cfg()
    r = np.random.default_rng(21)
    glob, doubles, singles = _flux_weights(r, cfg)
    lat, txt, cos_t, sin_t = _flux_inputs(r, cfg)
    got = blocks.flux_forward(cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t)
    return cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, got


def test_flux_forward_vs_float64(orc, flux_case):
    cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, got = flux_case
    ref = flux_f64(orc, cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t)
    err = rel_l2(got, ref)
    print(f"flux forward velocity: rel L2 {err:.2e}")
    assert err < FLUX_TOL


@pytest.mark.parametrize("mistake", FLUX_MISTAKES)
def test_flux_forward_catches_planted_mistake(orc, flux_case, mistake):
    cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, got = flux_case
    bad = flux_f64(orc, cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t, mistake=mistake)
    err = rel_l2(got, bad)
    print(f"{mistake}: rel L2 {err:.2e}")
    assert err > 10 * FLUX_TOL


def test_flux_forward_zero_gates_closed_form(orc):
    """Every double- and single-block gate at 0 makes each block the identity
    on its stream, so the velocity is
    unpatchify(final_linear(LN(img_in(patchify(latent))) * (1 + scale) + shift))
    with (shift, scale) = final_mod . silu(time_in1 . silu(time_in0 . temb))."""
    from oracle import blocks
    cfg = _flux_cfg()
    r = np.random.default_rng(22)
    glob, doubles, singles = _flux_weights(r, cfg, zero_gates=True)
    lat, txt, cos_t, sin_t = _flux_inputs(r, cfg)
    got = blocks.flux_forward(cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t)
    d = cfg.dim
    G = lambda b, wt, n, k: _deq(orc, b, wt, n, k)  # noqa: E731
    img = _patchify(lat.astype(np.float64), cfg.patch) @ G(glob["img_in"], Q8, d, cfg.patch_dim).T
    vec = _silu(_timestep(cfg.t_emb_dim, 500.0) @ G(glob["time_in0"], Q4K, d, cfg.t_emb_dim).T)
    vec = _silu(vec @ G(glob["time_in1"], Q4K, d, d).T)
    fm = (vec @ G(glob["final_mod"], Q4K, 2 * d, d).T).reshape(2, d)
    a = _ln(img, 1e-6) * (1.0 + fm[1]) + fm[0]
    ref = _unpatchify(a @ G(glob["final_linear"], Q4K, cfg.patch_dim, d).T, cfg.latent_ch, cfg.latent_h,
                      cfg.latent_w, cfg.patch)
    err = rel_l2(got, ref)
    print(f"zero-gate velocity vs closed form: rel L2 {err:.2e}")
    assert err < 1e-3


def test_flux_blocks_sampled_rows_match_full(orc, flux_case):
    """The sampled-row forms of the double and single block (used at full
    shape against the GPU) give the full block's rows bit for bit."""
    from oracle import blocks
    cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, _ = flux_case
    d, nt = cfg.dim, cfg.n_txt
    r = np.random.default_rng(23)
    txt_h = r.standard_normal((nt, d)).astype(np.float32)
    img = r.standard_normal((cfg.n_img, d)).astype(np.float32)
    mt, mi = (r.standard_normal((6, d)).astype(np.float32) for _ in range(2))
    w = doubles[0]
    ft, fi = blocks.flux_double_block(w, txt_h, img, mt, mi, cfg.n_heads, cos_t, sin_t)
    rows = np.array([0, 5, nt - 1, nt, nt + 17, nt + cfg.n_img - 1])
    part = blocks.flux_double_block(w, txt_h, img, mt, mi, cfg.n_heads, cos_t, sin_t, rows=rows)
    np.testing.assert_array_equal(part, np.concatenate([ft, fi])[rows])
    h = np.concatenate([txt_h, img])
    ms = r.standard_normal((3, d)).astype(np.float32)
    full = blocks.flux_single_block(singles[0], h, ms, cfg.n_heads, cos_t, sin_t)
    part = blocks.flux_single_block(singles[0], h, ms, cfg.n_heads, cos_t, sin_t, rows=rows)
    np.testing.assert_array_equal(part, full[rows])


def test_zimage_layer_sampled_rows_match_full(orc, zimage_case):
    """The sampled-row form of the Z-Image layer (used at full size against
    the GPU) gives the full layer's rows bit for bit."""
    from oracle import blocks
    w, h, H, cos_t, sin_t = zimage_case[:5]
    full = blocks.zimage_layer(w, h, H, cos_t, sin_t)
    rows = np.array([0, 3, 17, h.shape[0] // 2, h.shape[0] - 1])
    part = blocks.zimage_layer(w, h, H, cos_t, sin_t, rows=rows)
    np.testing.assert_array_equal(part, full[rows])


# ---------------------------------------------------------------------------
# the reference's own Flux.2 MLP form (SwiGLU halves)
# ---------------------------------------------------------------------------

FLUX_SWIGLU_MISTAKES = ["swiglu_halves", "swiglu_gelu", "swiglu_no_gate", "cat_order", "gate_chunks"]


@pytest.fixture(scope="module")
def flux_swiglu_case(orc):
    from oracle import blocks
    cfg = _flux_cfg("swiglu")
    r = np.random.default_rng(31)
    glob, doubles, singles = _flux_weights(r, cfg)
    lat, txt, cos_t, sin_t = _flux_inputs(r, cfg)
    got = blocks.flux_forward(cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t)
    return cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, got


def test_flux_swiglu_forward_vs_float64(orc, flux_swiglu_case):
    """The SwiGLU MLP form of both block types (linear1 [3 d + 2 m, d], MLP
    in-projection [2 m, d]) against the float64 restatement."""
    cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, got = flux_swiglu_case
    ref = flux_f64(orc, cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t)
    err = rel_l2(got, ref)
    print(f"flux (swiglu) forward velocity: rel L2 {err:.2e}")
    assert err < FLUX_TOL


@pytest.mark.parametrize("mistake", FLUX_SWIGLU_MISTAKES)
def test_flux_swiglu_forward_catches_planted_mistake(orc, flux_swiglu_case, mistake):
    cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, got = flux_swiglu_case
    bad = flux_f64(orc, cfg, glob, doubles, singles, lat, txt, 0.5, cos_t, sin_t, mistake=mistake)
    err = rel_l2(got, bad)
    print(f"{mistake}: rel L2 {err:.2e}")
    assert err > 10 * FLUX_TOL


def test_flux_swiglu_blocks_sampled_rows_match_full(orc, flux_swiglu_case):
    """The sampled-row forms of the SwiGLU blocks give the full blocks' rows
    bit for bit."""
    from oracle import blocks
    cfg, glob, doubles, singles, lat, txt, cos_t, sin_t, _ = flux_swiglu_case
    d, nt = cfg.dim, cfg.n_txt
    r = np.random.default_rng(33)
    txt_h = r.standard_normal((nt, d)).astype(np.float32)
    img = r.standard_normal((cfg.n_img, d)).astype(np.float32)
    mt, mi = (r.standard_normal((6, d)).astype(np.float32) for _ in range(2))
    ft, fi = blocks.flux_double_block(doubles[0], txt_h, img, mt, mi, cfg.n_heads, cos_t, sin_t, mlp_act="swiglu")
    rows = np.array([0, 5, nt - 1, nt, nt + 17, nt + cfg.n_img - 1])
    part = blocks.flux_double_block(doubles[0], txt_h, img, mt, mi, cfg.n_heads, cos_t, sin_t, rows=rows,
                                    mlp_act="swiglu")
    np.testing.assert_array_equal(part, np.concatenate([ft, fi])[rows])
    h = np.concatenate([txt_h, img])
    ms = r.standard_normal((3, d)).astype(np.float32)
    full = blocks.flux_single_block(singles[0], h, ms, cfg.n_heads, cos_t, sin_t, mlp_act="swiglu")
    part = blocks.flux_single_block(singles[0], h, ms, cfg.n_heads, cos_t, sin_t, rows=rows, mlp_act="swiglu")
    np.testing.assert_array_equal(part, full[rows])
