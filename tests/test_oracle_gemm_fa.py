"""Pins the oracle's GEMM, attention and RoPE restatements against float64
brute force, exact-answer constructions and invariants. CPU only."""
import math

import numpy as np
import pytest

from conftest import rel_l2
from llmr_amd import gguf, synth, workloads


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


@pytest.mark.parametrize("M,N,K", [(5, 7, 64), (9, 33, 256), (1, 3, 512)])
def test_q8_gemm_vs_float64(orc, M, N, K):
    w = synth.normal(1, 1, (N + 2) * K, 0.02)
    blk = gguf.quantize_q8_0(w)
    x = synth.normal(1, 2, M * K).reshape(M, K)
    got = orc.batch_matmul(blk, 8, x, N, K, M, row_offset=2)
    b = orc.dequant_q8_0_operand(blk).view(np.float16).astype(np.float64).reshape(N + 2, K)[2:]
    exp = _f16(x) @ b.T
    # only the f32 accumulation differs from float64 (products are exact)
    bound = K * 2.0**-24 * (np.abs(_f16(x)) @ np.abs(b).T) + 1e-30
    assert np.all(np.abs(got - exp) <= bound)
    assert rel_l2(got, exp) < 1e-5


@pytest.mark.parametrize("M,N,K", [(4, 6, 256), (7, 17, 768)])
def test_q4k_gemm_vs_float64(orc, M, N, K):
    w = synth.normal(2, 1, (N + 1) * K, 0.02)
    blk = gguf.quantize_q4k(w)
    x = synth.normal(2, 2, M * K).reshape(M, K)
    got = orc.batch_matmul(blk, 12, x, N, K, M, row_offset=1)
    b = orc.dequant_q4k(blk).astype(np.float64).reshape(N + 1, K)[1:]
    exp = x.astype(np.float64) @ b.T
    bound = 2 * K * 2.0**-24 * (np.abs(x) @ np.abs(b).T) + 1e-30
    assert np.all(np.abs(got - exp) <= bound)


def test_q8_gemm_identity_exact(orc):
    """W = I (scale 1/127, q = 127): each output is one exact product."""
    N = K = 64
    w = np.eye(N, K, dtype=np.float32)
    blk = gguf.quantize_q8_0(w)
    x = (np.arange(3 * K, dtype=np.float32).reshape(3, K) % 29 - 14) / 8.0
    got = orc.batch_matmul(blk, 8, x, N, K, 3)
    c = np.float32(np.float16(np.float16(1 / 127.0) * np.float16(127)))
    assert np.array_equal(got, x * c)


@pytest.mark.parametrize("wtype", [8, 12])
def test_gemm_row_offset_is_column_slice(orc, wtype):
    M, n, K = 3, 40, 256
    blk = gguf.quantize(synth.normal(3, 1, 3 * n * K, 0.02), wtype)
    x = synth.normal(3, 2, M * K).reshape(M, K)
    full = orc.batch_matmul(blk, wtype, x, 3 * n, K, M)
    for s in range(3):
        part = orc.batch_matmul(blk, wtype, x, n, K, M, row_offset=s * n)
        assert np.array_equal(part, full[:, s * n:(s + 1) * n])
    rows = orc.batch_matmul(blk, wtype, x, 3 * n, K, M, rows=[2, 0])
    assert np.array_equal(rows, full[[2, 0]])


def _silu64(g):
    return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("M,N,K", [(5, 7, 64), (3, 40, 320), (1, 9, 512)])
def test_swiglu_gemm_vs_float64(orc, M, N, K):
    """silu(x Wg^T) * (x Wu^T) with f32 activations and the exact f32 dequant
    (batch_matmul_swiglu_q8), against float64; a gate/up swap, a missing g
    factor (sigmoid instead of silu) or fp16-rounded operands all fail it."""
    wg = gguf.quantize_q8_0(synth.normal(4, 1, N * K, 0.05))
    wu = gguf.quantize_q8_0(synth.normal(4, 2, N * K, 0.05))
    x = synth.normal(4, 3, M * K).reshape(M, K)
    got = orc.batch_matmul_swiglu_q8(wg, wu, x, N, K, M)
    bg = orc.dequant_q8_0(wg).astype(np.float64).reshape(N, K)
    bu = orc.dequant_q8_0(wu).astype(np.float64).reshape(N, K)
    x64 = x.astype(np.float64)
    g, u = x64 @ bg.T, x64 @ bu.T
    exp = _silu64(g) * u
    # f32 accumulation of K products each rounded once, then silu and the product
    eg = 2 * K * 2.0**-24 * (np.abs(x64) @ np.abs(bg).T)
    eu = 2 * K * 2.0**-24 * (np.abs(x64) @ np.abs(bu).T)
    bound = eg * np.abs(u) * 1.2 + eu * np.abs(_silu64(g)) + 8 * 2.0**-24 * np.abs(exp) + 1e-30
    assert np.all(np.abs(got - exp) <= bound)
    for wrong in (_silu64(u) * g, g / (1.0 + np.exp(-g)) / np.where(g == 0, 1, g) * u):
        assert rel_l2(got, wrong) > 1e-2
    rows = orc.batch_matmul_swiglu_q8(wg, wu, x, N, K, M, rows=[M - 1, 0])
    assert np.array_equal(rows, got[[M - 1, 0]])


def test_swiglu_special_values(orc):
    """g = 0 gives 0 whatever u; a large negative g gives -0 * u; u = 0 gives 0."""
    N, K = 4, 32
    w0 = np.zeros((N, K), np.float32)
    wg = w0.copy()
    wg[1, 0] = -60.0  # g = -60 x0
    wg[2, 0] = 1.0
    wu = np.ones((N, K), np.float32)
    wu[2] = 0.0
    x = np.zeros((1, K), np.float32)
    x[0, 0] = 1.0
    got = orc.batch_matmul_swiglu_q8(gguf.quantize_q8_0(wg), gguf.quantize_q8_0(wu), x, N, K, 1)[0]
    assert got[0] == 0.0 and got[2] == 0.0 and got[3] == 0.0
    assert abs(got[1]) < 1e-20


def _attn64(q, k, v, scale):
    q, k, v = (_f16(t) for t in (q, k, v))
    H, S, D = q.shape
    s = np.einsum("hsd,htd->hst", q, k) * scale
    s -= s.max(axis=2, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=2, keepdims=True)
    o = np.einsum("hst,htd->hsd", p, v)
    return np.transpose(o, (1, 0, 2)).reshape(S, H * D)


@pytest.mark.parametrize("H,S", [(1, 1), (2, 31), (1, 32), (2, 70), (1, 200)])
def test_fa_vs_float64(orc, H, S):
    n = H * S * 128
    q = synth.normal(4, 1, n).reshape(H, S, 128)
    k = synth.normal(4, 2, n).reshape(H, S, 128)
    v = synth.normal(4, 3, n).reshape(H, S, 128)
    got = orc.flash_attention(q, k, v, 1 / math.sqrt(128))
    exp = _attn64(q, k, v, 1 / math.sqrt(128))
    assert rel_l2(got, exp) < 2e-6


def test_fa_invariants(orc):
    H, S = 2, 100
    n = H * S * 128
    q = synth.normal(5, 1, n).reshape(H, S, 128) * 2
    k = synth.normal(5, 2, n).reshape(H, S, 128) * 2
    base = synth.normal(5, 3, H * 128).reshape(H, 1, 128).astype(np.float16).astype(np.float32)
    v = np.repeat(base, S, axis=1)
    o = orc.flash_attention(q, k, v, 0.1).reshape(S, H, 128)
    assert np.allclose(o, np.transpose(v, (1, 0, 2)), rtol=1e-6, atol=1e-6)
    v2 = synth.normal(5, 4, n).reshape(H, S, 128)
    perm = np.random.default_rng(1).permutation(S)
    o1 = orc.flash_attention(q, k, v2, 0.1)
    o2 = orc.flash_attention(q, k[:, perm], v2[:, perm], 0.1)
    assert rel_l2(o2, o1) < 1e-6
    # sampled query range / heads equal the full computation
    part = orc.flash_attention(q, k, v2, 0.1, heads=(1, 2), qrange=(32, 64))
    assert np.array_equal(part.reshape(S, H, 128)[32:64, 1], o1.reshape(S, H, 128)[32:64, 1])


def test_rope_tables_and_rotation(orc):
    a = workloads.FLUX_ATTENTION
    pos = workloads.attention_positions(a)
    c, s = orc.rope_tables(pos, a.axes, a.theta)
    # closed form in float64
    pair = 0
    for ai, dims in enumerate(a.axes):
        for kk in range(dims // 2):
            ang = pos[:, ai].astype(np.float64) * a.theta ** (-2.0 * kk / dims)
            assert np.max(np.abs(c[:, pair] - np.cos(ang))) < 2e-5
            assert np.max(np.abs(s[:, pair] - np.sin(ang))) < 2e-5
            pair += 1
    assert pair == 64
    # product-side tables agree with the oracle's
    pc, ps = workloads.rope_tables(pos, a.axes, a.theta)
    assert np.max(np.abs(pc - c)) < 1e-5 and np.max(np.abs(ps - s)) < 1e-5
    x = synth.normal(6, 1, 2 * a.S * 128).reshape(2, a.S, 128)
    y = orc.rope_apply(x, c, s)
    nx = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    ny = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert np.allclose(nx, ny, rtol=1e-5, atol=1e-6)
    assert np.array_equal(y[:, : a.n_txt], x[:, : a.n_txt])  # text ids are all zero: identity
    py = workloads.rope_apply(x, pc, ps)
    assert np.max(np.abs(py - y)) < 1e-4
