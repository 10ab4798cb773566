"""GGUF block formats used by the hot path: type ids, sizes and quantizers.

Block layouts (raw GGUF, exactly what the reference uploads to the device,
lib/model/tensor.c3:48-66):
  Q8_0  32 weights in 34 bytes: f16 scale d, then 32 int8 q; w = d*q
        (lib/gguf/types.c3:58,83,100-103; lib/model/tensor.c3:354-361).
  Q4_K  256 weights in 144 bytes: f16 d @0, f16 dmin @2, 12 packed 6-bit
        (scale, min) pairs @4, 128 bytes of nibbles @16; element j*64+h*32+l
        is nibble h of qs[j*32+l], w = d*sc*q - dmin*mn
        (lib/gguf/types.c3:62,87; lib/model/tensor.c3:292-335).
Rows are stored back to back with no padding ([N, K] row-major, ne = [K, N],
tools/gguf_writer.py:12-14).
"""
from __future__ import annotations

import numpy as np

GGML_F32 = 0
GGML_F16 = 1
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_BF16 = 30

# (block_size, type_size): lib/gguf/types.c3:50-98
_SIZES = {
    GGML_F32: (1, 4),
    GGML_F16: (1, 2),
    GGML_Q8_0: (32, 34),
    GGML_Q4_K: (256, 144),
    GGML_BF16: (1, 2),
}

TYPE_NAMES = {GGML_F32: "F32", GGML_F16: "F16", GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K",
              GGML_BF16: "BF16"}


def block_size(t: int) -> int:
    return _SIZES[t][0]


def type_size(t: int) -> int:
    return _SIZES[t][1]


def row_bytes(t: int, n: int) -> int:
    bs, ts = _SIZES[t]
    if n % bs:
        raise ValueError(f"{TYPE_NAMES.get(t, t)} row of {n} elements is not whole blocks of {bs}")
    return n // bs * ts


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """Q8_0 quantizer with the rule of tools/gguf_writer.py:121-157.

    Per 32-element block in float64: amax = max|v|, d = amax/127 (floored at
    1e-8), scale stored as one round-to-nearest-even float64->float16 rounding
    (struct '<e'), q = floor(v/d + 0.5) for v >= 0 and -floor(-v/d + 0.5)
    otherwise (half away from zero) using the unrounded d, clamped to +-127.
    Returns the raw block bytes (uint8, n/32*34)."""
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 32).astype(np.float64)
    nb = v.shape[0]
    amax = np.abs(v).max(axis=1)
    d = amax / 127.0
    d = np.where(d < 1e-8, 1e-8, d)
    inv = 1.0 / d
    dh = d.astype(np.float16)
    t = v * inv[:, None]
    q = np.where(v >= 0, np.floor(t + 0.5), -np.floor(-t + 0.5))
    q = np.clip(q, -127, 127).astype(np.int8)
    out = np.empty((nb, 34), np.uint8)
    out[:, 0:2] = dh.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def quantize_q4k(x: np.ndarray) -> np.ndarray:
    """Q4_K quantizer (this project's own rule; the reference ships none,
    tools/gguf_writer.py:51-60,160-169).

    Per 256-element superblock in float64: for each 32-element sub-block s,
    mn_s = max(0, -min), sc_s = (max + mn_s)/15; d = max(sc)/63 and
    dmin = max(mn)/63 stored as RNE halves; 6-bit ls = round(sc_s/d),
    lm = round(mn_s/dmin); q = round((v + dmin*lm)/(d*ls)) clamped to [0,15];
    round(x) = floor(x + 0.5). The 12 scale bytes are the inverse of
    get_scale_min_k4 (llm.slang:447-462). Returns raw block bytes (n/256*144)."""
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8, 32).astype(np.float64)
    nb = v.shape[0]
    lo = v.min(axis=2)
    hi = v.max(axis=2)
    mn = np.where(lo < 0, -lo, 0.0)
    sc = (hi + mn) / 15.0
    dmax = np.maximum(sc.max(axis=1), 0.0)
    mmax = np.maximum(mn.max(axis=1), 0.0)
    dbits = (dmax / 63.0).astype(np.float16)
    mbits = (mmax / 63.0).astype(np.float16)
    dd = dbits.astype(np.float64)[:, None]
    dm = mbits.astype(np.float64)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        ls = np.where(dd > 0, np.clip(np.floor(sc / dd + 0.5), 0, 63), 0).astype(np.uint32)
        lm = np.where(dm > 0, np.clip(np.floor(mn / dm + 0.5), 0, 63), 0).astype(np.uint32)
        S = (dd * ls)[:, :, None]
        O = (dm * lm)[:, :, None]
        q = np.where(S > 0, np.clip(np.floor((v + O) / S + 0.5), 0, 15), 0).astype(np.uint8)
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = dbits.view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = mbits.view(np.uint8).reshape(nb, 2)
    for j in range(4):
        out[:, 4 + j] = ((ls[:, j] & 63) | ((ls[:, j + 4] >> 4) << 6)).astype(np.uint8)
        out[:, 8 + j] = ((lm[:, j] & 63) | ((lm[:, j + 4] >> 4) << 6)).astype(np.uint8)
        out[:, 12 + j] = ((ls[:, j + 4] & 15) | ((lm[:, j + 4] & 15) << 4)).astype(np.uint8)
    qq = q.reshape(nb, 4, 2, 32)  # [j][h][l]
    out[:, 16:] = (qq[:, :, 0, :] | (qq[:, :, 1, :] << 4)).reshape(nb, 128)
    return out.reshape(-1)


def quantize(x: np.ndarray, t: int) -> np.ndarray:
    if t == GGML_Q8_0:
        return quantize_q8_0(x)
    if t == GGML_Q4_K:
        return quantize_q4k(x)
    raise ValueError(f"no quantizer for ggml type {t}")
