"""GPU dequant vs the oracle: bit-exact (f32 and fp16 operand forms)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _exhaustive_q8_blocks():
    scales = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    nb = 65536 * 8
    blk = np.zeros((nb, 34), np.uint8)
    blk[:, 0:2] = np.repeat(scales, 8).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = np.tile(q.reshape(8, 32), (65536, 1)).view(np.uint8)
    return blk


def _bits_eq_nan(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    fa = a.view(np.float32) if a.dtype == np.float32 else a.view(np.float16).astype(np.float32)
    fb = b.view(np.float32) if b.dtype == np.float32 else b.view(np.float16).astype(np.float32)
    na, nb = np.isnan(fa), np.isnan(fb)
    return np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb])


@pytest.mark.parametrize("rows_per_tensor", [64])
def test_q8_0_dequant_exhaustive(orc, dev, rows_per_tensor):
    import torch
    from llmr_amd import ops
    blk = _exhaustive_q8_blocks()  # 524288 blocks: all scales x all int8
    K = blk.shape[0] // rows_per_tensor * 32
    w = torch.from_numpy(blk.reshape(-1)).to(dev)
    got = ops.dequant(w, 8, rows_per_tensor, K).cpu().numpy().reshape(-1)
    exp = orc.dequant_q8_0(blk)
    assert _bits_eq_nan(got, exp)
    got16 = ops.dequant_operand_f16(w, 8, rows_per_tensor, K).cpu().numpy().view(np.uint16).reshape(-1)
    exp16 = orc.dequant_q8_0_operand(blk)
    assert _bits_eq_nan(got16, exp16)


def test_q8_0_dequant_row_offset(orc, dev):
    import torch
    from llmr_amd import ops, gguf, synth
    N, K = 40, 96
    x = synth.normal(7, 1, N * K, 0.02)
    blk = gguf.quantize_q8_0(x)
    w = torch.from_numpy(blk).to(dev)
    got = ops.dequant(w, 8, 13, K, row_offset=17).cpu().numpy()
    exp = orc.dequant_q8_0(blk).reshape(N, K)[17:30]
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_q4k_dequant_random_and_special(orc, dev):
    import torch
    from llmr_amd import ops
    rng = np.random.default_rng(11)
    nb = 4096
    blk = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    # d, dmin over all exponent classes incl. subnormal, Inf and NaN patterns
    dm = rng.integers(0, 65536, size=(nb, 2), dtype=np.uint32).astype(np.uint16)
    blk[:, 0:4] = dm.view(np.uint8).reshape(nb, 4)
    K = 256 * 16
    w = torch.from_numpy(blk.reshape(-1)).to(dev)
    got = ops.dequant(w, 12, nb // 16, K).cpu().numpy().reshape(-1)
    exp = orc.dequant_q4k(blk)
    assert _bits_eq_nan(got, exp)
    got16 = ops.dequant_operand_f16(w, 12, nb // 16, K).cpu().numpy().view(np.uint16).reshape(-1)
    exp16 = orc.dequant_q4k_operand(blk)
    fin = np.isfinite(exp) & (np.abs(exp) < 65504)
    bad = np.nonzero(fin & (got16 != exp16))[0]
    for i in bad[:12]:
        print(f"elem {i}: f32 {exp[i]!r} ({exp[i:i+1].view(np.uint32)[0]:#010x}) "
              f"gpu {got16[i]:#06x} oracle {exp16[i]:#06x}")
    print(f"{bad.size} mismatches of {int(fin.sum())}")
    assert bad.size == 0


def test_q4k_dequant_flux_weight_slice(orc, dev):
    import torch
    from llmr_amd import ops, gguf, synth
    N, K = 96, 3072
    x = synth.normal(42, 7, N * K, 0.02)
    blk = gguf.quantize_q4k(x)
    w = torch.from_numpy(blk).to(dev)
    got = ops.dequant(w, 12, 64, K, row_offset=32).cpu().numpy()
    exp = orc.dequant_q4k(blk).reshape(N, K)[32:96]
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
