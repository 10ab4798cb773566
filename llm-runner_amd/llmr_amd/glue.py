"""Torch-tensor front end of the block-glue entry points of libllmr_hip.so.

Each function takes device tensors (2-D views with unit column stride are
fine: a row range such as hidden[n_txt:] or a column slice such as
l1[:, 3*dim:] is passed by pointer and row stride, with no copy) and issues
one C-ABI call on the graph's stream. The ops restate the reference's glue
dispatches (dependencies/zimage.c3l/shaders/zimage.slang, mrope.slang,
lib/shaders/diffusion.slang); the chains the reference runs as several
dispatches over one tensor are single calls here, as listed per function.
"""
from __future__ import annotations

import torch

from . import capi
from .gguf import GGML_BF16, GGML_F16, GGML_F32
from .ops import RenderGraph, default_graph

_GGML = {torch.float32: GGML_F32, torch.float16: GGML_F16, torch.bfloat16: GGML_BF16}


def _rows(t: torch.Tensor, what: str, dtype=None):
    """(pointer, row stride in elements) of a 2-D device view with unit column stride."""
    if not t.is_cuda:
        raise ValueError(f"{what} must be a device tensor")
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{what} must be a 2-D view with contiguous rows")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{what} must be {dtype}")
    return t.data_ptr(), t.stride(0) if t.shape[0] > 1 else t.shape[1] + (-t.shape[1]) % 4


def _vec(t, what: str, n: int):
    if t is None:
        return None
    if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous() or t.numel() < n:
        raise ValueError(f"{what} must be a contiguous f32 device vector of >= {n} elements")
    return t.data_ptr()


def _otype(t: torch.Tensor) -> int:
    if t.dtype not in _GGML:
        raise ValueError(f"unsupported output dtype {t.dtype}")
    return _GGML[t.dtype]


def batch_rmsnorm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, eps: float,
                  mod_scale: torch.Tensor | None = None, mod_shift: torch.Tensor | None = None,
                  g: RenderGraph | None = None) -> torch.Tensor:
    """out = rmsnorm(x) * weight [* (1 + mod_scale)] [+ mod_shift], out in its own dtype.
    batch_rmsnorm + scale_modulate (dependencies/zimage.c3l/dit.c3:1424-1432)."""
    g = g or default_graph()
    rows, dim = x.shape
    if out.shape != x.shape:
        raise ValueError("out must have x's shape")
    xp, xs = _rows(x, "x", torch.float32)
    op, os_ = _rows(out, "out")
    g.bind_stream()
    g.ctx.batch_rmsnorm(xp, xs, _vec(weight, "weight", dim), _vec(mod_scale, "mod_scale", dim),
                        _vec(mod_shift, "mod_shift", dim), op, _otype(out), os_, dim, rows, eps)
    return out


def batch_layernorm(x: torch.Tensor, out: torch.Tensor, eps: float, mod_scale: torch.Tensor | None = None,
                    mod_shift: torch.Tensor | None = None, g: RenderGraph | None = None) -> torch.Tensor:
    """out = layernorm(x) [* (1 + mod_scale)] [+ mod_shift]: batch_layernorm + adaln_modulate
    (dependencies/flux.c3l/flux_dit.c3:767-770)."""
    g = g or default_graph()
    rows, dim = x.shape
    if out.shape != x.shape:
        raise ValueError("out must have x's shape")
    xp, xs = _rows(x, "x", torch.float32)
    op, os_ = _rows(out, "out")
    g.bind_stream()
    g.ctx.batch_layernorm(xp, xs, _vec(mod_scale, "mod_scale", dim), _vec(mod_shift, "mod_shift", dim), op,
                          _otype(out), os_, dim, rows, eps)
    return out


def batch_layernorm_split(x: torch.Tensor, out: torch.Tensor, eps: float, split_row: int, mods, mods2,
                          g: RenderGraph | None = None) -> torch.Tensor:
    """batch_layernorm of rows from two streams in one launch: rows
    [0, split_row) modulated by mods = (mod_scale, mod_shift), the rest by
    mods2 (either vector may be None; split_row % 4 == 0); the rows equal
    two batch_layernorm calls' (the Flux double block's text and image
    LayerNorms, dependencies/flux.c3l/flux_dit.c3:761-779)."""
    g = g or default_graph()
    rows, dim = x.shape
    if out.shape != x.shape:
        raise ValueError("out must have x's shape")
    xp, xs = _rows(x, "x", torch.float32)
    op, os_ = _rows(out, "out")
    g.bind_stream()
    g.ctx.batch_layernorm_split(xp, xs, _vec(mods[0], "mod_scale", dim), _vec(mods[1], "mod_shift", dim), split_row,
                                _vec(mods2[0], "mod_scale2", dim), _vec(mods2[1], "mod_shift2", dim), op, _otype(out),
                                os_, dim, rows, eps)
    return out


def qkv_heads(qkv: torch.Tensor, n_heads: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              row0: int = 0, q_norm: torch.Tensor | None = None, k_norm: torch.Tensor | None = None,
              eps: float = 1e-6, rope: tuple | None = None, g: RenderGraph | None = None) -> None:
    """Rows of a QKV GEMM output (f32 [rows, >= 3*n_heads*128], Q | K | V from
    column 0) -> head norm, RoPE and head-major q/k/v [n_heads, seq, 128] at
    sequence rows row0 .. row0+rows (batch_head_norm + transpose_heads + mrope,
    dependencies/flux.c3l/flux_dit.c3:814-863)."""
    g = g or default_graph()
    rows = qkv.shape[0]
    sp, ss = _rows(qkv, "qkv", torch.float32)
    H, S, D = q.shape
    if D != 128 or H != n_heads or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q/k/v must be [n_heads, seq, 128] alike")
    if not (q.dtype == k.dtype == v.dtype) or not all(t.is_contiguous() and t.is_cuda for t in (q, k, v)):
        raise ValueError("q/k/v must be contiguous device tensors of one dtype")
    cos_p = sin_p = None
    if rope is not None:
        cos_t, sin_t = rope
        cos_p = _vec(cos_t, "rope_cos", S * 64)
        sin_p = _vec(sin_t, "rope_sin", S * 64)
    g.bind_stream()
    g.ctx.qkv_heads(sp, ss, rows, n_heads, _vec(q_norm, "q_norm", 128), _vec(k_norm, "k_norm", 128), eps,
                    cos_p, sin_p, q.data_ptr(), k.data_ptr(), v.data_ptr(), _otype(q), S, row0)


def gated_residual(residual: torch.Tensor, inp: torch.Tensor, gate: torch.Tensor | None = None,
                   mode: int = capi.GATE_LINEAR, norm_weight: torch.Tensor | None = None, eps: float = 1e-5,
                   g: RenderGraph | None = None) -> torch.Tensor:
    """residual += gate(d) * [rmsnorm](inp): gated_residual_linear / gated_residual (tanh) /
    residual_add, with the Z-Image post-norm fused (dependencies/zimage.c3l/dit.c3:1495-1503)."""
    g = g or default_graph()
    rows, dim = residual.shape
    if inp.shape != residual.shape:
        raise ValueError("input must have the residual's shape")
    hp, hs = _rows(residual, "residual", torch.float32)
    xp, xs = _rows(inp, "input", torch.float32)
    g.bind_stream()
    g.ctx.gated_residual(hp, hs, xp, xs, _vec(norm_weight, "norm_weight", dim), _vec(gate, "gate", dim), mode,
                         dim, rows, eps)
    return residual


def gated_residual_rmsnorm(residual: torch.Tensor, inp: torch.Tensor, gate: torch.Tensor | None, mode: int,
                           norm_weight: torch.Tensor | None, eps: float, next_weight: torch.Tensor,
                           out: torch.Tensor, next_eps: float, mod_scale: torch.Tensor | None = None,
                           mod_shift: torch.Tensor | None = None, g: RenderGraph | None = None) -> torch.Tensor:
    """gated_residual, then batch_rmsnorm of the updated residual (next_weight,
    mod_scale, mod_shift, next_eps) into out, in one pass: the Z-Image
    block's attention post-norm + gated residual and its FFN pre-norm
    (dependencies/zimage.c3l/dit.c3:1495-1503, 1545-1554); bit for bit the
    two calls. dim <= 4096."""
    g = g or default_graph()
    rows, dim = residual.shape
    if inp.shape != residual.shape or out.shape != residual.shape:
        raise ValueError("input and out must have the residual's shape")
    hp, hs = _rows(residual, "residual", torch.float32)
    xp, xs = _rows(inp, "input", torch.float32)
    op, os_ = _rows(out, "out")
    g.bind_stream()
    g.ctx.gated_residual_rmsnorm(hp, hs, xp, xs, _vec(norm_weight, "norm_weight", dim), _vec(gate, "gate", dim),
                                 mode, _vec(next_weight, "next_weight", dim), _vec(mod_scale, "mod_scale", dim),
                                 _vec(mod_shift, "mod_shift", dim), op, _otype(out), os_, dim, rows, eps, next_eps)
    return out


def activation(src: torch.Tensor, dst: torch.Tensor, act: int, src2: torch.Tensor | None = None,
               g: RenderGraph | None = None) -> torch.Tensor:
    """dst = act(src) (ACT_SILU_MUL: silu(src) * src2), dst in its own dtype; src and src2 are
    column slices of one f32 buffer, dst a column slice of another (silu, gelu, elemwise_mul,
    concat_rows_copy: dependencies/flux.c3l/flux_dit.c3:1051-1057)."""
    g = g or default_graph()
    rows, cols = src.shape
    if dst.shape != src.shape:
        raise ValueError("dst must have src's shape")
    sp, ss = _rows(src, "src", torch.float32)
    dp, ds = _rows(dst, "dst")
    src2_col = 0
    if act == capi.ACT_SILU_MUL:
        if src2 is None or src2.shape != src.shape:
            raise ValueError("ACT_SILU_MUL needs src2 of src's shape")
        p2, s2 = _rows(src2, "src2", torch.float32)
        off = p2 - sp
        if s2 != ss or off < 0 or off % 16:  # bytes; the column offset must be a multiple of 4
            raise ValueError("src2 must be a column slice of src's buffer at or after src")
        src2_col = off // 4
    g.bind_stream()
    # the views' pointers already include their column offsets, so the
    # library's column offsets are 0 (src) and the distance to src2
    if rows == 1:  # a single row has no real stride; give the library one that covers it
        ss = max(ss, src2_col + cols + (-(src2_col + cols)) % 4)
        ds = max(ds, cols + (-cols) % 4)
    g.ctx.activation(sp, ss, 0, src2_col, dp, _otype(dst), ds, 0, rows, cols, act)
    return dst


def timestep_embed(out: torch.Tensor, t: float, g: RenderGraph | None = None) -> torch.Tensor:
    g = g or default_graph()
    g.bind_stream()
    g.ctx.timestep_embed(_vec(out, "out", out.numel()), out.numel(), t)
    return out


def patchify(latent: torch.Tensor, out: torch.Tensor, patch: int, g: RenderGraph | None = None) -> torch.Tensor:
    g = g or default_graph()
    C, H, W = latent.shape
    if latent.dtype != torch.float32 or not latent.is_contiguous() or not out.is_contiguous():
        raise ValueError("latent must be contiguous f32, out contiguous")
    if out.numel() != C * H * W:
        raise ValueError("out must hold C*H*W elements")
    g.bind_stream()
    g.ctx.patchify(latent.data_ptr(), out.data_ptr(), _otype(out), C, H, W, patch)
    return out


def unpatchify(patches: torch.Tensor, out: torch.Tensor, patch: int, g: RenderGraph | None = None) -> torch.Tensor:
    g = g or default_graph()
    C, H, W = out.shape
    if patches.dtype != torch.float32 or out.dtype != torch.float32:
        raise ValueError("unpatchify is f32")
    if not patches.is_contiguous() or not out.is_contiguous() or patches.numel() != out.numel():
        raise ValueError("patches and out must be contiguous with C*H*W elements")
    g.bind_stream()
    g.ctx.unpatchify(patches.data_ptr(), out.data_ptr(), C, H, W, patch)
    return out


def synth_q4k(n_rows: int, in_dim: int, stream: int, std: float = 0.02, seed: int = 42,
              device="cuda", g: RenderGraph | None = None) -> torch.Tensor:
    """Raw Q4_K blocks of an [n_rows, in_dim] weight ~N(0, std^2), generated on the device."""
    g = g or default_graph()
    out = torch.empty(n_rows * (in_dim // 256) * 144, dtype=torch.uint8, device=device)
    g.bind_stream()
    g.ctx.synth_q4k(out.data_ptr(), n_rows, in_dim, seed, stream, std)
    return out
