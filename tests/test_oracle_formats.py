"""Pins the oracle's format arithmetic (fp16 conversions, GGUF block decode,
quantizers) against numpy's IEEE conversions, exhaustive sweeps and blocks
built from known fields. CPU only."""
import numpy as np
import pytest

from llmr_amd import gguf


def _nan_eq(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equality of f32 arrays, any NaN equal to any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def test_f16_decode_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(bits)
    exp = bits.view(np.float16).astype(np.float32)
    e31 = ((bits >> 10) & 0x1F) == 31
    # reference quirk: exponent 31 -> +-Inf for Inf and NaN (llm.slang:245-247)
    exp[e31] = np.where((bits[e31] >> 15) != 0, -np.inf, np.inf).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def _f16_midpoints():
    """f32 values halfway between consecutive finite halves, and their neighbours."""
    h = np.arange(0, 0x7BFF, dtype=np.uint16)  # finite positive halves except the max
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in f32
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(0))
    v = np.concatenate([mid, up, dn])
    return np.concatenate([v, -v])


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(1)
    rand = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                        2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001, 2.0**-26, 1e-45, 6.0e-8,
                        2.0**-14, 2.0**-14 * (1 - 2.0**-11)], np.float32)
    x = np.concatenate([rand, _f16_midpoints(), special])
    x = x[~np.isnan(x)]
    got = orc.f32_to_f16(x)
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)
    nan = orc.f32_to_f16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_f64_to_f16_single_rounding(orc):
    rng = np.random.default_rng(2)
    x = np.exp(rng.uniform(np.log(1e-9), np.log(7e4), 20000))
    h = np.arange(1, 0x7BFF, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    h2 = (np.arange(1, 0x7BFF, 7, dtype=np.uint16) + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = (h + h2) / 2
    # just above a midpoint in f64 but the same as the midpoint once in f32:
    # a double rounding through f32 would round these to even instead of up
    tricky = mid * (1 + 2.0**-40)
    vals = np.concatenate([x, mid, tricky, [0.0, 1e-8, 65504.0, 65519.0]])
    got = np.array([orc.f64_to_f16(v) for v in vals], np.uint16)
    exp = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


def _pack_scales(ls, lm):
    """Layout of the 12 Q4_K scale bytes as documented for GGML Q4_K: bytes 0-3
    hold sc[0..3] (6 bits) + the top 2 bits of sc[4..7]; bytes 4-7 mn[0..3] + top
    2 bits of mn[4..7]; bytes 8-11 the low nibbles of sc[4..7] | mn[4..7] << 4."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (ls[j] & 63) | ((ls[j + 4] >> 4) << 6)
        s[j + 4] = (lm[j] & 63) | ((lm[j + 4] >> 4) << 6)
        s[j + 8] = (ls[j + 4] & 15) | ((lm[j + 4] & 15) << 4)
    return s


def test_get_scale_min_k4_roundtrip(orc):
    rng = np.random.default_rng(3)
    for _ in range(3000):
        ls = rng.integers(0, 64, 8)
        lm = rng.integers(0, 64, 8)
        s = _pack_scales(ls, lm)
        for i in range(8):
            assert orc.get_scale_min_k4(i, s) == (ls[i], lm[i])


def test_q8_0_dequant_exhaustive(orc):
    scales = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)  # 256 values = 8 blocks
    nb = 65536 * 8
    blk = np.zeros((nb, 34), np.uint8)
    blk[:, 0:2] = np.repeat(scales, 8).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = np.tile(q.reshape(8, 32), (65536, 1)).view(np.uint8)
    got = orc.dequant_q8_0(blk)
    d = np.repeat(scales, 8).view(np.float16).astype(np.float32)
    e31 = ((np.repeat(scales, 8) >> 10) & 0x1F) == 31
    d[e31] = np.where((np.repeat(scales, 8)[e31] >> 15) != 0, -np.inf, np.inf)
    with np.errstate(invalid="ignore"):
        exp = (d[:, None] * np.tile(q.reshape(8, 32), (65536, 1)).astype(np.float32)).reshape(-1)
    assert _nan_eq(got, exp)

    # the fp16 operand: one IEEE fp16 multiply of the (NaN->Inf) scale and q
    got16 = orc.dequant_q8_0_operand(blk)
    with np.errstate(invalid="ignore", over="ignore"):
        exp16 = (d.astype(np.float16)[:, None]
                 * np.tile(q.reshape(8, 32), (65536, 1)).astype(np.float16)).reshape(-1)
    assert _nan_eq(got16.view(np.float16).astype(np.float32), exp16.astype(np.float32))


SPECIAL_D = [0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x2A3F, 0x1234, 0x7BFF, 0x7C00, 0xFC00]


@pytest.mark.parametrize("dbits,mbits", [(a, b) for a in SPECIAL_D for b in (0x0000, 0x0001, 0x2A3F, 0x7BFF, 0x7C00)]
                         + [(0x2E66, 0x1C29), (0x1F00, 0x2200)])
def test_q4k_dequant_from_known_fields(orc, dbits, mbits):
    """Blocks built from known (d, dmin, sc, mn, q): every (sc, mn) pair, every q."""
    pairs = [(sc, mn) for sc in range(64) for mn in range(64)]
    nb = len(pairs) // 8
    blk = np.zeros((nb, 144), np.uint8)
    exp = np.zeros((nb, 256), np.float64)
    d = float(np.uint16(dbits).view(np.float16))
    dm = float(np.uint16(mbits).view(np.float16))
    if np.isnan(d):
        d = np.copysign(np.inf, d)
    l = np.arange(32)
    for b in range(nb):
        ls = np.array([pairs[8 * b + s][0] for s in range(8)])
        lm = np.array([pairs[8 * b + s][1] for s in range(8)])
        qv = np.zeros(256, np.uint8)
        for s in range(8):
            qv[32 * s:32 * s + 32] = (l + 3 * s + b) % 16
        blk[b, 0:2] = np.array([dbits], np.uint16).view(np.uint8)
        blk[b, 2:4] = np.array([mbits], np.uint16).view(np.uint8)
        blk[b, 4:16] = _pack_scales(ls, lm)
        for j in range(4):
            blk[b, 16 + 32 * j:16 + 32 * j + 32] = qv[64 * j:64 * j + 32] | (qv[64 * j + 32:64 * j + 64] << 4)
        with np.errstate(invalid="ignore"):
            for s in range(8):
                a = d * ls[s] * qv[32 * s:32 * s + 32].astype(np.float64)
                c = dm * lm[s]
                e = a - c
                if np.all(np.isfinite(e)):
                    # the f64 difference must be exact for the f32 rounding below to be the single
                    # rounding the reference performs
                    assert np.all((e + c) - a == 0)
                exp[b, 32 * s:32 * s + 32] = e
    got = orc.dequant_q4k(blk)
    with np.errstate(invalid="ignore", over="ignore"):
        assert _nan_eq(got, exp.reshape(-1).astype(np.float32))


def test_q8_0_quantizer_known_answers(orc):
    x = np.zeros(96, np.float32)
    x[32] = 127.0
    x[33], x[34], x[35], x[36] = 2.5, -2.5, 0.4999, -126.5
    x[64:96] = np.linspace(-1, 1, 32, dtype=np.float32) * 1e-3
    b = orc.quantize_q8_0(x).reshape(3, 34)
    assert b[0, 0] == 0 and b[0, 1] == 0 and not b[0, 2:].any()  # d = 1e-8 rounds to +0
    assert (b[1, 0], b[1, 1]) == (0x00, 0x3C)  # d = 1.0
    q = b[1, 2:].view(np.int8)
    assert list(q[:5]) == [127, 3, -3, 0, -127]  # half away from zero, clamp at 127
    assert np.array_equal(b, gguf.quantize_q8_0(x).reshape(3, 34))


def test_q8_0_quantizer_matches_product_and_bounds(orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(32 * 4096) * 0.02).astype(np.float32)
    x[:64] *= 1e-6
    c = orc.quantize_q8_0(x)
    p = gguf.quantize_q8_0(x)
    assert np.array_equal(c, p)
    deq = orc.dequant_q8_0(c).astype(np.float64)
    xb = x.astype(np.float64).reshape(-1, 32)
    d = np.maximum(np.abs(xb).max(1) / 127.0, 1e-8)
    d16 = c.reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    bound = 0.5 * d + 127 * np.abs(d16 - d) + 1e-12
    assert np.all(np.abs(deq.reshape(-1, 32) - xb) <= bound[:, None] * (1 + 1e-9))


def test_q4k_quantizer_matches_product_and_bounds(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(256 * 2048) * 0.02).astype(np.float32)
    x[:256] = np.abs(x[:256])          # all-positive superblock (mn = 0)
    x[256:512] = -np.abs(x[256:512])   # all-negative superblock
    x[512:768] = 0.0                   # all-zero superblock
    c = orc.quantize_q4k(x)
    p = gguf.quantize_q4k(x)
    assert np.array_equal(c, p)
    deq = orc.dequant_q4k(c).astype(np.float64).reshape(-1, 32)
    xs = x.astype(np.float64).reshape(-1, 32)
    rng_s = xs.max(1) - np.minimum(xs.min(1), 0)
    err = np.abs(deq - xs).max(1)
    assert np.all(err <= rng_s / 15 * 0.75 + 1e-7)
    assert np.sqrt(np.mean((deq - xs) ** 2)) < 0.15 * np.std(xs)


def _nearest_half_exact(v):
    """binary16 bits nearest to the rational v (ties to even), by exact comparison."""
    from fractions import Fraction
    if abs(v) >= 65520:
        return 0xFC00 if v < 0 else 0x7C00
    h = int(np.array([float(v)], np.float64).astype(np.float16).view(np.uint16)[0])
    best = None
    for c in (h - 1, h, h + 1, (h ^ 0x8000)):
        c &= 0xFFFF
        if (c & 0x7C00) == 0x7C00:
            continue
        cv = Fraction(float(np.uint16(c).view(np.float16)))
        key = (abs(cv - v), (c & 1))
        if best is None or key < best[0]:
            best = (key, c)
    b = best[1]
    return 0 if (b == 0x8000 and v >= 0) else b


def test_q4k_operand_single_rounding_exact(orc):
    """The Q4_K fp16 operand is the exact d*sc*q - dmin*mn rounded once; blocks
    with d, dmin chosen so that many exact values sit on or next to f16 ties."""
    from fractions import Fraction
    rng = np.random.default_rng(12)
    nb = 96
    blk = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    dbits = rng.integers(0x3800, 0x7000, size=nb).astype(np.uint16)
    mbits = np.where(rng.random(nb) < 0.5, rng.integers(0x0001, 0x0400, size=nb),
                     rng.integers(0x1000, 0x5000, size=nb)).astype(np.uint16)
    blk[:, 0:2] = dbits.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = mbits.view(np.uint8).reshape(nb, 2)
    got = orc.dequant_q4k_operand(blk).reshape(nb, 256)
    for b in range(nb):
        d = Fraction(float(dbits[b].view(np.float16)))
        dm = Fraction(float(mbits[b].view(np.float16)))
        for e in range(0, 256, 3):
            j, h, l = e >> 6, (e >> 5) & 1, e & 31
            sc, mn = orc.get_scale_min_k4(2 * j + h, blk[b, 4:16])
            q = (int(blk[b, 16 + 32 * j + l]) >> (4 * h)) & 15
            exact = d * sc * q - dm * mn
            assert got[b, e] == _nearest_half_exact(exact), (b, e, float(exact))
