"""Deterministic synthetic inputs: counter-based SplitMix64 -> Box-Muller.

Every tensor of a workload is one stream identified by (seed, stream); element
i of a stream depends only on (seed, stream, i), so any slice can be
regenerated independently (a test can rebuild rows 1000..1015 of a 4608-row
activation without the rest). The base seed 42 is the reference's default
(dependencies/flux.c3l/pipeline.c3:64); the generator itself is this
project's own (the reference's latent RNG, lib/pipelines/scheduler.c3:78-99,
is not on the hot path).
"""
from __future__ import annotations

import os

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
BASE_SEED = 42


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> np.uint64:
    """64-bit key of stream `stream` under `seed`."""
    with np.errstate(over="ignore"):
        z = np.array([(seed * 0x100000001B3 + stream * 0x632BE59BD9B4E019) & (2**64 - 1)],
                     dtype=np.uint64)
        return _mix(z)[0]


def uniform_bits(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """SplitMix64 outputs with counters start..start+count-1."""
    key = stream_key(seed, stream)
    with np.errstate(over="ignore"):
        idx = np.arange(start, start + count, dtype=np.uint64) + np.uint64(1)
        return _mix(key + idx * _GOLDEN)


_CHUNK = 1 << 22  # elements per worker task (even)


def normal(seed: int, stream: int, count: int, std: float = 1.0, start: int = 0) -> np.ndarray:
    """`count` N(0, std^2) samples (f32) of elements start..start+count-1.

    Element 2j is r*cos(2*pi*u2), element 2j+1 is r*sin(2*pi*u2) with
    r = sqrt(-2 ln(1 - u1)), u1 and u2 taken from counters 2j and 2j+1 (53-bit
    uniforms), all in float64, scaled by std and rounded once to f32.
    Large requests are split over a thread pool (numpy releases the GIL);
    the result does not depend on the split.
    """
    if count > 2 * _CHUNK:
        from concurrent.futures import ThreadPoolExecutor
        out = np.empty(count, np.float32)
        starts = list(range(0, count, _CHUNK))

        def work(o):
            n = min(_CHUNK, count - o)
            out[o:o + n] = _normal_block(seed, stream, n, std, start + o)

        with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
            list(ex.map(work, starts))
        return out
    return _normal_block(seed, stream, count, std, start)


def _normal_block(seed: int, stream: int, count: int, std: float, start: int) -> np.ndarray:
    j0 = start // 2
    j1 = (start + count + 1) // 2
    bits = uniform_bits(seed, stream, 2 * j0, 2 * (j1 - j0)).reshape(-1, 2)
    u = (bits >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
    th = 2.0 * np.pi * u[:, 1]
    z = np.empty((j1 - j0) * 2, np.float64)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    off = start - 2 * j0
    return (z[off:off + count] * std).astype(np.float32)


def normal_rows(seed: int, stream: int, n_cols: int, rows, std: float = 1.0) -> np.ndarray:
    """Rows `rows` of a [*, n_cols] row-major tensor drawn by `normal`."""
    rows = list(rows)
    out = np.empty((len(rows), n_cols), np.float32)
    for i, r in enumerate(rows):
        out[i] = normal(seed, stream, n_cols, std, start=int(r) * n_cols)
    return out
