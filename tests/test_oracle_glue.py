"""The oracle's block-glue restatements pinned against float64 closed forms.

Each check is chosen so that a plausible restatement mistake fails it: a
dropped eps (tiny inputs), one-pass variance (large mean), the wrong
reduction axis, erf-GELU instead of the tanh form, sin/cos halves swapped,
a transposed patch layout."""
import math

import numpy as np
import pytest

from conftest import rel_l2


def _rng(seed=0):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("dim", [100, 256, 3072, 3840])
def test_rmsnorm_closed_form(orc, dim):
    r = _rng(dim)
    x = r.standard_normal((7, dim)).astype(np.float32)
    x[3] *= 1e-4  # eps dominates this row: a dropped eps fails here
    w = (1 + 0.1 * r.standard_normal(dim)).astype(np.float32)
    eps = 1e-5
    y = orc.batch_rmsnorm(x, w, eps)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + eps) * w
    assert np.abs(y - ref).max() <= 4e-6 * np.abs(ref).max()
    bad = xd / np.sqrt((xd ** 2).mean(1, keepdims=True)) * w
    assert np.abs(y[3] - bad[3]).max() > 1e-2 * np.abs(bad[3]).max()


@pytest.mark.parametrize("dim", [128, 3072])
def test_layernorm_closed_form(orc, dim):
    r = _rng(dim + 1)
    x = (r.standard_normal((5, dim)) + 300.0).astype(np.float32)  # large mean: one-pass variance cancels
    eps = 1e-6
    y = orc.batch_layernorm(x, eps)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + eps)
    assert rel_l2(y, ref) < 1e-4  # f32 x - mean at |x| ~ 300 carries ~ulp(300) = 3e-5
    # the f32 one-pass form E[x^2] - E[x]^2 is far off at this mean
    xf = x.astype(np.float32)
    var1 = (xf * xf).mean(1, keepdims=True, dtype=np.float32) - xf.mean(1, keepdims=True, dtype=np.float32) ** 2
    one_pass = (xd - mu) / np.sqrt(np.abs(var1.astype(np.float64)) + eps)
    assert rel_l2(one_pass, ref) > 1e-3


def test_modulate_forms(orc):
    r = _rng(2)
    x = r.standard_normal((4, 64)).astype(np.float32)
    sc = r.standard_normal(64).astype(np.float32)
    sh = r.standard_normal(64).astype(np.float32)
    np.testing.assert_array_equal(orc.modulate(x, sc), (x * (np.float32(1) + sc)).astype(np.float32))
    np.testing.assert_array_equal(orc.modulate(x, sc, sh), (x * (np.float32(1) + sc) + sh).astype(np.float32))


def test_head_norm_per_head(orc):
    r = _rng(3)
    H, S = 3, 5
    x = r.standard_normal((S, H * 128)).astype(np.float32)
    x[:, 128:256] *= 10.0  # heads of different scale: normalising over the row would fail
    w = (1 + 0.1 * r.standard_normal(128)).astype(np.float32)
    y = orc.batch_head_norm(x, w, H, 1e-6)
    xd = x.reshape(S, H, 128).astype(np.float64)
    ref = (xd / np.sqrt((xd ** 2).mean(2, keepdims=True) + 1e-6) * w).reshape(S, H * 128)
    assert np.abs(y - ref).max() < 1e-5


def test_transpose_heads_layout(orc):
    S, H = 6, 3
    x = np.arange(S * H * 128, dtype=np.float32).reshape(S, H * 128)
    y = orc.transpose_heads(x, H)
    np.testing.assert_array_equal(y, x.reshape(S, H, 128).transpose(1, 0, 2))


def test_gated_residual_forms(orc):
    r = _rng(4)
    res = r.standard_normal((3, 32)).astype(np.float32)
    g = r.standard_normal(32).astype(np.float32)
    x = r.standard_normal((3, 32)).astype(np.float32)
    lin = orc.gated_residual(res, g, x, False)
    np.testing.assert_allclose(lin, res.astype(np.float64) + g * x.astype(np.float64), rtol=0, atol=1e-6)
    th = orc.gated_residual(res, g, x, True)
    np.testing.assert_allclose(th, res + np.tanh(g.astype(np.float64)) * x, rtol=0, atol=2e-6)
    # the clip threshold bounds each update
    big = np.full((1, 32), 1e3, np.float32)
    clipped = orc.gated_residual(np.zeros((1, 32), np.float32), np.full(32, 5.0, np.float32), big, True,
                                 clip_thresh=10.0)
    np.testing.assert_array_equal(clipped, np.full((1, 32), 10.0, np.float32))


def test_silu_gelu_closed_forms(orc):
    x = np.linspace(-12, 12, 4001, dtype=np.float32)
    xd = x.astype(np.float64)
    np.testing.assert_allclose(orc.silu(x), xd / (1 + np.exp(-xd)), rtol=2e-6, atol=1e-7)
    gel = 0.5 * xd * (1 + np.tanh(0.7978845608 * (xd + 0.044715 * xd ** 3)))
    np.testing.assert_allclose(orc.gelu(x), gel, rtol=2e-6, atol=1e-6)
    erf_gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xd])
    assert np.abs(orc.gelu(x) - erf_gelu).max() > 1e-4  # the tanh form, not the erf form


def test_timestep_embed_closed_form(orc):
    dim, t = 256, 500.0
    y = orc.timestep_embed(dim, t)
    half = dim // 2
    j = np.arange(half, dtype=np.float64)
    freq = np.exp(-math.log(10000.0) * j / half)
    ref = np.concatenate([np.cos(t * freq), np.sin(t * freq)])
    assert np.abs(y - ref).max() < 5e-4  # f32 argument t*freq up to 500: ulp(500) ~ 3e-5 rad
    assert y[0] == pytest.approx(math.cos(t)) and y[half] == pytest.approx(math.sin(t), abs=1e-4)


def test_patchify_layout_and_roundtrip(orc):
    r = _rng(5)
    C, H, W, p = 3, 8, 12, 2
    x = r.standard_normal((C, H, W)).astype(np.float32)
    y = orc.patchify(x, p)
    ref = x.reshape(C, H // p, p, W // p, p).transpose(1, 3, 2, 4, 0).reshape((H // p) * (W // p), p * p * C)
    np.testing.assert_array_equal(y, ref)
    np.testing.assert_array_equal(orc.unpatchify(y, C, H, W, p), x)


def test_zimage_layer_zero_gates_is_identity(orc):
    """With both adaLN gates at 0, tanh(0) = 0 makes the layer the identity."""
    from oracle import blocks
    from llmr_amd import gguf
    r = _rng(6)
    dim, H, ffn, S = 256, 2, 512, 40

    def q8(n, k):
        return gguf.quantize((0.02 * r.standard_normal((n, k))).astype(np.float32), gguf.GGML_Q8_0)
    one = np.ones(dim, np.float32)
    w = dict(wqkv=q8(3 * dim, dim), wo=q8(dim, dim), w_gate=q8(ffn, dim), w_up=q8(ffn, dim), w_down=q8(dim, ffn),
             attn_norm1=one, attn_norm2=one, ffn_norm1=one, ffn_norm2=one, q_norm=np.ones(128, np.float32),
             k_norm=np.ones(128, np.float32), adaln=np.zeros((4, dim), np.float32))
    h = r.standard_normal((S, dim)).astype(np.float32)
    cos_t = np.ones((S, 64), np.float32)
    sin_t = np.zeros((S, 64), np.float32)
    np.testing.assert_array_equal(blocks.zimage_layer(w, h, H, cos_t, sin_t), h)
    w["adaln"][1] = 1.0
    assert np.abs(blocks.zimage_layer(w, h, H, cos_t, sin_t) - h).max() > 1e-3
