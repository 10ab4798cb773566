"""The oracle's LoRA restatements (two-hop correction, Q8_0 merge) pinned
against what the mathematics fixes.

* Integer-valued operands make every f32 sum exact, so the hops must equal the
  int64 products exactly: a transposed A or B, a wrong row offset or a wrong
  weight-row offset fails.
* Float data: within f32 rounding of a float64 product.
* A zero update leaves a Q8_0 weight quantized by the reference rule
  byte-identical (d*q is exact, absmax = 127 d, u / d = q).
* The requantized block is within half a step (plus the f16 rounding of the
  stored scale) of the exact updated values, and its scale is absmax / 127.
"""
import numpy as np
import pytest

from conftest import rel_l2


def _ints(r, shape, lo=-3, hi=4):
    return r.integers(lo, hi, size=shape).astype(np.float32)


def test_lora_down_exact_on_integers(orc):
    r = np.random.default_rng(1)
    A = _ints(r, (24, 700))
    X = _ints(r, (9, 700))
    got = orc.lora_down(A, X)
    np.testing.assert_array_equal(got, (X.astype(np.int64) @ A.T.astype(np.int64)).astype(np.float32))


def test_lora_down_float_close_to_float64(orc):
    r = np.random.default_rng(2)
    A = r.standard_normal((16, 3072)).astype(np.float32)
    X = r.standard_normal((5, 3072)).astype(np.float32)
    ref = X.astype(np.float64) @ A.T.astype(np.float64)
    got = orc.lora_down(A, X)
    bound = 3072 * 2.0 ** -24 * (np.abs(X).astype(np.float64) @ np.abs(A).T.astype(np.float64))
    assert np.all(np.abs(got - ref) <= bound)


def test_lora_up_exact_placement(orc):
    r = np.random.default_rng(3)
    seq, rank, out_dim, b_rows, row_off, w_off = 7, 5, 64, 20, 30, 11
    B = _ints(r, (w_off + b_rows + 4, rank))
    s = _ints(r, (seq, rank))
    y0 = _ints(r, (seq, out_dim), -50, 50)
    got = orc.lora_up(B, s, y0, 0.5, row_offset=row_off, weight_row_offset=w_off, b_rows=b_rows)
    ref = y0.astype(np.float64).copy()
    ref[:, row_off:row_off + b_rows] += 0.5 * (s.astype(np.int64) @ B[w_off:w_off + b_rows].T.astype(np.int64))
    np.testing.assert_array_equal(got, ref.astype(np.float32))


def test_lora_up_float_close_to_float64(orc):
    r = np.random.default_rng(4)
    B = r.standard_normal((300, 32)).astype(np.float32)
    s = r.standard_normal((6, 32)).astype(np.float32)
    y0 = r.standard_normal((6, 300)).astype(np.float32)
    got = orc.lora_up(B, s, y0, 0.25)
    ref = y0.astype(np.float64) + 0.25 * (s.astype(np.float64) @ B.T.astype(np.float64))
    assert rel_l2(got, ref) < 1e-6


def _q8_weight(r, rows, in_dim, std=0.05):
    from llmr_amd import gguf
    return gguf.quantize((std * r.standard_normal((rows, in_dim))).astype(np.float32), gguf.GGML_Q8_0)


def test_q8_merge_zero_update_is_identity(orc):
    r = np.random.default_rng(5)
    w = _q8_weight(r, 12, 512)
    w2 = w.reshape(12, -1).copy()
    w2[3] = 0  # an all-zero row: d = 0, stays 0 (1e-8 rounds to f16 zero)
    A = np.zeros((4, 512), np.float32)
    B = r.standard_normal((12, 4)).astype(np.float32)
    np.testing.assert_array_equal(orc.q8_lora_merge(w2, A, B, 512, 1.0), w2.reshape(-1))
    A = r.standard_normal((4, 512)).astype(np.float32)
    np.testing.assert_array_equal(orc.q8_lora_merge(w2, A, B, 512, 0.0), w2.reshape(-1))


def test_q8_merge_requant_bounds_and_untouched_rows(orc):
    r = np.random.default_rng(6)
    rows, in_dim, rank, off, b_rows = 20, 768, 8, 5, 9
    w = _q8_weight(r, rows, in_dim)
    A = (0.1 * r.standard_normal((rank, in_dim))).astype(np.float32)
    B = (0.1 * r.standard_normal((b_rows, rank))).astype(np.float32)
    scale = 0.75
    got = orc.q8_lora_merge(w, A, B, in_dim, scale, dst_row_offset=off)
    row_bytes = in_dim // 32 * 34
    g2, w2 = got.reshape(rows, row_bytes), w.reshape(rows, row_bytes)
    np.testing.assert_array_equal(g2[:off], w2[:off])
    np.testing.assert_array_equal(g2[off + b_rows:], w2[off + b_rows:])
    base = orc.dequant_q8_0(w2[off:off + b_rows].reshape(-1)).reshape(b_rows, in_dim)
    u = base.astype(np.float64) + scale * (B.astype(np.float64) @ A.astype(np.float64))
    merged = orc.dequant_q8_0(g2[off:off + b_rows].reshape(-1)).reshape(b_rows, in_dim).astype(np.float64)
    ub = np.abs(u).reshape(b_rows, in_dim // 32, 32)
    dn = ub.max(axis=2) / 127.0
    sbits = g2[off:off + b_rows].reshape(b_rows, in_dim // 32, 34)[:, :, :2].copy().view(np.uint16)[..., 0]
    d16 = orc.f16_to_f32(sbits).astype(np.float64)
    # stored scale: f16 of absmax / 127 (one f16 rounding; the f32 absmax and
    # division add a few f32 ulps)
    assert np.all(np.abs(d16 - dn) <= 2.0 ** -11 * dn + 1e-12)
    # each element within half a step of the exact update (+ scale rounding
    # times 127, + f32 rounding of the update)
    err = np.abs(merged - u).reshape(b_rows, in_dim // 32, 32)
    tol = 0.5 * dn + 127 * np.abs(d16 - dn) + 1e-6 * ub.max(axis=2)
    assert np.all(err <= tol[..., None])


def test_q8_merge_saturates_and_rounds_half_away(orc):
    """One block whose update dominates: q' = round(127 u / absmax) with
    halves away from zero, the extremes at +-127."""
    in_dim = 256
    w = np.zeros(in_dim // 32 * 34, np.uint8)
    A = np.zeros((1, in_dim), np.float32)
    vals = np.array([254.0, -254.0, 1.0, -1.0, 3.0, -3.0, 0.0, 127.0] * 4, np.float32)  # block 0
    A[0, :32] = vals
    B = np.ones((1, 1), np.float32)
    got = orc.q8_lora_merge(w, A, B, in_dim, 1.0)
    q = got[2:34].view(np.int8)
    # d' = 254/127 = 2: 254 -> 127, 1 -> 0.5 -> 1 (away from zero), 3 -> 1.5 -> 2, 127 -> 63.5 -> 64
    np.testing.assert_array_equal(q[:8], np.array([127, -127, 1, -1, 2, -2, 0, 64], np.int8))
    assert got[:2].copy().view(np.uint16)[0] == 0x4000  # f16 2.0
