"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP backend. Imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the product.
The C restatement and its reference citations live in oracle/oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t


def build() -> str:
    """Compile liboracle.so from oracle.c (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f16_to_f32_n": (None, [_u16p, _sz, _f32p]),
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f32_to_f16_n": (None, [_f32p, _sz, _u16p]),
            "orc_f64_to_f16": (ctypes.c_uint16, [ctypes.c_double]),
            "orc_get_scale_min_k4": (None, [_u32, _u8p, _u32p, _u32p]),
            "orc_dequant_q8_0": (None, [_u8p, _sz, _f32p]),
            "orc_dequant_q4k": (None, [_u8p, _sz, _f32p]),
            "orc_dequant_q8_0_operand": (None, [_u8p, _sz, _u16p]),
            "orc_dequant_q4k_operand": (None, [_u8p, _sz, _u16p]),
            "orc_quantize_q8_0": (None, [_f32p, _sz, _u8p]),
            "orc_quantize_q4k": (None, [_f32p, _sz, _u8p]),
            "orc_batch_matmul_q8": (None, [_u8p, _f32p, _f32p, _u32, _u32, _u32, _u32]),
            "orc_batch_matmul_q4k": (None, [_u8p, _f32p, _f32p, _u32, _u32, _u32, _u32]),
            "orc_batch_matmul_q8_rows": (None, [_u8p, _f32p, _f32p, _u32, _u32, _u32, _u32, _u32p, _u32]),
            "orc_batch_matmul_swiglu_q8": (None, [_u8p, _u8p, _f32p, _f32p, _u32, _u32, _u32]),
            "orc_batch_matmul_swiglu_q8_rows": (None, [_u8p, _u8p, _f32p, _f32p, _u32, _u32, _u32, _u32p, _u32]),
            "orc_batch_matmul_q4k_rows": (None, [_u8p, _f32p, _f32p, _u32, _u32, _u32, _u32, _u32p, _u32]),
            "orc_flash_attention": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32, ctypes.c_float,
                                           _u32, _u32, _u32, _u32]),
            "orc_rope_tables": (None, [_u32p, _u32, _u32p, _u32, ctypes.c_float, _f32p, _f32p]),
            "orc_lora_down": (None, [_f32p, _f32p, _f32p, _u32, _u32, _u32]),
            "orc_lora_up": (None, [_f32p, _f32p, _f32p, _u32, _u32, _u32, ctypes.c_float, _u32, _u32, _u32]),
            "orc_q8_lora_merge": (None, [_u8p, _f32p, _f32p, _u32, _u32, _u32, _u32, ctypes.c_float]),
            "orc_rope_apply": (None, [_f32p, _u32, _u32, _f32p, _f32p]),
            "orc_num_threads": (ctypes.c_int, []),
            "orc_batch_rmsnorm": (None, [_f32p, _f32p, _f32p, _u32, _u32, ctypes.c_float]),
            "orc_batch_layernorm": (None, [_f32p, _f32p, _u32, _u32, ctypes.c_float]),
            "orc_modulate": (None, [_f32p, _f32p, _f32p, _u32, _sz]),
            "orc_batch_head_norm": (None, [_f32p, _f32p, _u32, _u32, _u32, ctypes.c_float]),
            "orc_transpose_heads": (None, [_f32p, _f32p, _u32, _u32, _u32]),
            "orc_gated_residual": (None, [_f32p, _f32p, _f32p, _u32, _sz, ctypes.c_int, ctypes.c_float,
                                          ctypes.c_float]),
            "orc_silu": (None, [_f32p, _sz]),
            "orc_gelu": (None, [_f32p, _sz]),
            "orc_timestep_embed": (None, [_f32p, _u32, ctypes.c_float]),
            "orc_patchify": (None, [_f32p, _f32p, _u32, _u32, _u32, _u32]),
            "orc_unpatchify": (None, [_f32p, _f32p, _u32, _u32, _u32, _u32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray, ptype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ptype)


def num_threads() -> int:
    return lib().orc_num_threads()


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_f16_to_f32_n(_p(bits, _u16p), bits.size, _p(out, _f32p))
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(x, _f32p), x.size, _p(out, _u16p))
    return out


def f64_to_f16(x: float) -> int:
    return int(lib().orc_f64_to_f16(float(x)))


def get_scale_min_k4(is_: int, scales12: np.ndarray):
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc, mn = ctypes.c_uint32(), ctypes.c_uint32()
    lib().orc_get_scale_min_k4(is_, _p(s, _u8p), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


def dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    n = b.size // 34
    out = np.empty(n * 32, np.float32)
    lib().orc_dequant_q8_0(_p(b, _u8p), n, _p(out, _f32p))
    return out


def dequant_q8_0_operand(blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    n = b.size // 34
    out = np.empty(n * 32, np.uint16)
    lib().orc_dequant_q8_0_operand(_p(b, _u8p), n, _p(out, _u16p))
    return out


def dequant_q4k(blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    n = b.size // 144
    out = np.empty(n * 256, np.float32)
    lib().orc_dequant_q4k(_p(b, _u8p), n, _p(out, _f32p))
    return out


def dequant_q4k_operand(blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    n = b.size // 144
    out = np.empty(n * 256, np.uint16)
    lib().orc_dequant_q4k_operand(_p(b, _u8p), n, _p(out, _u16p))
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0(_p(x, _f32p), x.size, _p(out, _u8p))
    return out


def quantize_q4k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // 256 * 144, np.uint8)
    lib().orc_quantize_q4k(_p(x, _f32p), x.size, _p(out, _u8p))
    return out


def batch_matmul(W: np.ndarray, wtype: int, X: np.ndarray, out_dim: int, in_dim: int,
                 seq_len: int, row_offset: int = 0, rows=None) -> np.ndarray:
    """Reference GEMM (wtype 8 = Q8_0, 12 = Q4_K) on f32 activations X [seq_len, in_dim].
    With `rows`, only those output rows are computed (result [len(rows), out_dim])."""
    W = np.ascontiguousarray(W, dtype=np.uint8).reshape(-1)
    X = np.ascontiguousarray(X, dtype=np.float32)
    assert X.size == seq_len * in_dim
    L = lib()
    if rows is None:
        Y = np.empty((seq_len, out_dim), np.float32)
        fn = L.orc_batch_matmul_q8 if wtype == 8 else L.orc_batch_matmul_q4k
        fn(_p(W, _u8p), _p(X, _f32p), _p(Y, _f32p), out_dim, in_dim, seq_len, row_offset)
        return Y
    r = np.ascontiguousarray(rows, dtype=np.uint32)
    if r.size and int(r.max()) >= seq_len:
        raise ValueError(f"sampled row {int(r.max())} >= seq_len {seq_len}")
    Y = np.empty((r.size, out_dim), np.float32)
    fn = L.orc_batch_matmul_q8_rows if wtype == 8 else L.orc_batch_matmul_q4k_rows
    fn(_p(W, _u8p), _p(X, _f32p), _p(Y, _f32p), out_dim, in_dim, seq_len, row_offset,
       _p(r, _u32p), r.size)
    return Y


def batch_matmul_swiglu_q8(Wg: np.ndarray, Wu: np.ndarray, X: np.ndarray, out_dim: int, in_dim: int,
                           seq_len: int, rows=None) -> np.ndarray:
    """Reference SwiGLU GEMM (batch_matmul_swiglu_q8, llm.slang:1769-1911) on f32
    activations X [seq_len, in_dim] and Q8_0 gate/up weights [out_dim, in_dim].
    With `rows`, only those output rows are computed (result [len(rows), out_dim])."""
    Wg = np.ascontiguousarray(Wg, dtype=np.uint8).reshape(-1)
    Wu = np.ascontiguousarray(Wu, dtype=np.uint8).reshape(-1)
    X = np.ascontiguousarray(X, dtype=np.float32)
    assert X.size == seq_len * in_dim
    L = lib()
    if rows is None:
        Y = np.empty((seq_len, out_dim), np.float32)
        L.orc_batch_matmul_swiglu_q8(_p(Wg, _u8p), _p(Wu, _u8p), _p(X, _f32p), _p(Y, _f32p), out_dim, in_dim,
                                     seq_len)
        return Y
    r = np.ascontiguousarray(rows, dtype=np.uint32)
    if r.size and int(r.max()) >= seq_len:
        raise ValueError(f"sampled row {int(r.max())} >= seq_len {seq_len}")
    Y = np.empty((r.size, out_dim), np.float32)
    L.orc_batch_matmul_swiglu_q8_rows(_p(Wg, _u8p), _p(Wu, _u8p), _p(X, _f32p), _p(Y, _f32p), out_dim, in_dim,
                                      seq_len, _p(r, _u32p), r.size)
    return Y


def flash_attention(Q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float,
                    heads=None, qrange=None) -> np.ndarray:
    """Reference attention on f32 [H, S, 128] inputs; returns O f32 [S, H*128]
    (entries outside the sampled heads / query range are NaN)."""
    H, S, D = Q.shape
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    K = np.ascontiguousarray(K, dtype=np.float32)
    V = np.ascontiguousarray(V, dtype=np.float32)
    O = np.full((S, H * D), np.nan, np.float32)
    h0, h1 = heads if heads is not None else (0, H)
    q0, q1 = qrange if qrange is not None else (0, S)
    lib().orc_flash_attention(_p(Q, _f32p), _p(K, _f32p), _p(V, _f32p), _p(O, _f32p), D, H, S,
                              float(scale), h0, h1, q0, q1)
    return O


def rope_tables(pos: np.ndarray, axes_dims, theta: float):
    pos = np.ascontiguousarray(pos, dtype=np.uint32)
    S, n_axes = pos.shape
    axes = np.ascontiguousarray(axes_dims, dtype=np.uint32)
    cos_t = np.zeros((S, 64), np.float32)
    sin_t = np.zeros((S, 64), np.float32)
    lib().orc_rope_tables(_p(pos, _u32p), S, _p(axes, _u32p), n_axes, float(theta),
                          _p(cos_t, _f32p), _p(sin_t, _f32p))
    return cos_t, sin_t


def rope_apply(x: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    H, S, D = x.shape
    assert D == 128
    lib().orc_rope_apply(_p(x, _f32p), H, S, _p(np.ascontiguousarray(cos_t, np.float32), _f32p),
                         _p(np.ascontiguousarray(sin_t, np.float32), _f32p))
    return x


# --- DiT block glue: one function per reference dispatch (f32 in, f32 out) ---

def _f32c(a) -> np.ndarray:
    return np.array(a, dtype=np.float32, copy=True, order="C")


def batch_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """batch_rmsnorm (zimage.slang:449-500) on [rows, dim]."""
    x = _f32c(x)
    rows, dim = x.shape
    out = np.empty_like(x)
    lib().orc_batch_rmsnorm(_p(x, _f32p), _p(_f32c(w), _f32p), _p(out, _f32p), dim, rows, float(eps))
    return out


def batch_layernorm(x: np.ndarray, eps: float) -> np.ndarray:
    """batch_layernorm (zimage.slang:502-561) on [rows, dim]."""
    x = _f32c(x)
    rows, dim = x.shape
    out = np.empty_like(x)
    lib().orc_batch_layernorm(_p(x, _f32p), _p(out, _f32p), dim, rows, float(eps))
    return out


def modulate(x: np.ndarray, scale: np.ndarray, shift=None) -> np.ndarray:
    """scale_modulate (shift None) / adaln_modulate over the last axis."""
    x = _f32c(x)
    dim = x.shape[-1]
    sh = _f32c(shift) if shift is not None else None
    lib().orc_modulate(_p(x, _f32p), _p(_f32c(scale), _f32p), _p(sh, _f32p) if sh is not None else None,
                       dim, x.size)
    return x


def batch_head_norm(x: np.ndarray, w: np.ndarray, n_heads: int, eps: float) -> np.ndarray:
    """batch_head_norm (zimage.slang:609-667) on [seq, n_heads*D]."""
    x = _f32c(x)
    S = x.shape[0]
    D = x.shape[1] // n_heads
    lib().orc_batch_head_norm(_p(x, _f32p), _p(_f32c(w), _f32p), n_heads, D, S, float(eps))
    return x


def transpose_heads(x: np.ndarray, n_heads: int) -> np.ndarray:
    """transpose_heads direction 0: [S, H*D] -> [H, S, D]."""
    x = _f32c(x)
    S = x.shape[0]
    D = x.shape[1] // n_heads
    out = np.empty((n_heads, S, D), np.float32)
    lib().orc_transpose_heads(_p(x, _f32p), _p(out, _f32p), S, n_heads, D)
    return out


def gated_residual(residual: np.ndarray, gate: np.ndarray, inp: np.ndarray, tanh_gate: bool,
                   scale: float = 1.0, clip_thresh: float = 0.0) -> np.ndarray:
    """gated_residual (tanh_gate) / gated_residual_linear; returns the updated residual."""
    r = _f32c(residual)
    x = _f32c(inp)
    lib().orc_gated_residual(_p(r, _f32p), _p(_f32c(gate), _f32p), _p(x, _f32p), r.shape[-1], r.size,
                             1 if tanh_gate else 0, float(scale), float(clip_thresh))
    return r


def silu(x: np.ndarray) -> np.ndarray:
    x = _f32c(x)
    lib().orc_silu(_p(x, _f32p), x.size)
    return x


def gelu(x: np.ndarray) -> np.ndarray:
    x = _f32c(x)
    lib().orc_gelu(_p(x, _f32p), x.size)
    return x


def timestep_embed(dim: int, t: float) -> np.ndarray:
    out = np.empty(dim, np.float32)
    lib().orc_timestep_embed(_p(out, _f32p), dim, float(t))
    return out


def patchify(latent: np.ndarray, ps: int) -> np.ndarray:
    x = _f32c(latent)
    C, H, W = x.shape
    out = np.empty(((H // ps) * (W // ps), C * ps * ps), np.float32)
    lib().orc_patchify(_p(x, _f32p), _p(out, _f32p), C, H, W, ps)
    return out


def unpatchify(patches: np.ndarray, C: int, H: int, W: int, ps: int) -> np.ndarray:
    x = _f32c(patches)
    out = np.empty((C, H, W), np.float32)
    lib().orc_unpatchify(_p(x, _f32p), _p(out, _f32p), C, H, W, ps)
    return out


def lora_down(A: np.ndarray, X: np.ndarray) -> np.ndarray:
    """LoRA hop 1: scratch [seq, rank] = X [seq, in_dim] . A [rank, in_dim]^T."""
    A = _f32c(A)
    X = _f32c(X)
    rank, in_dim = A.shape
    out = np.empty((X.shape[0], rank), np.float32)
    lib().orc_lora_down(_p(A, _f32p), _p(X, _f32p), _p(out, _f32p), rank, in_dim, X.shape[0])
    return out


def lora_up(B: np.ndarray, scratch: np.ndarray, out: np.ndarray, scale: float, row_offset: int = 0,
            weight_row_offset: int = 0, b_rows: int | None = None) -> np.ndarray:
    """LoRA hop 2 on a copy of `out` [seq, out_dim]; returns the updated copy."""
    B = _f32c(B)
    s = _f32c(scratch)
    y = np.array(out, dtype=np.float32, copy=True, order="C")
    rank = s.shape[1]
    b_rows = B.shape[0] - weight_row_offset if b_rows is None else b_rows
    lib().orc_lora_up(_p(B, _f32p), _p(s, _f32p), _p(y, _f32p), rank, y.shape[1], y.shape[0], float(scale),
                      row_offset, weight_row_offset, b_rows)
    return y


def q8_lora_merge(base: np.ndarray, A: np.ndarray, B: np.ndarray, in_dim: int, scale: float,
                  dst_row_offset: int = 0) -> np.ndarray:
    """Merged copy of Q8_0 blocks `base` (uint8, rows of in_dim/32 blocks)."""
    out = np.array(base, dtype=np.uint8, copy=True, order="C").reshape(-1)
    A = _f32c(A)
    B = _f32c(B)
    lib().orc_q8_lora_merge(_p(out, _u8p), _p(A, _f32p), _p(B, _f32p), in_dim, B.shape[0], dst_row_offset,
                            A.shape[0], float(scale))
    return out
