"""Workload shapes of the DiT hot path and their synthetic inputs.

Shapes are in GEMM form: M = tokens (seq_len), N = out_dim, K = in_dim.
  q8_linear       single Q8_0 linear, f32 activations [256, 3072], W [3072, 3072]
  flux_attention  non-causal attention, H=24, S=4608 (512 text + 4096 image), D=128,
                  f16 Q/K/V with Flux 3-axis RoPE (axes 16/56/56, theta 1e4)
                  applied beforehand
  flux_linear1    Flux single-stream fused QKV+MLP-in, Q4_K, bf16 [4608, 3072] -> 21504
  flux_linear2    Flux single-stream output projection, Q4_K, bf16 [4608, 15360] -> 3072
  flux_linear1_f32, flux_linear2_f32
                  the same with f32 activations (the reference's activation type)
  zimage_*        Z-Image block GEMMs (Q8_0, bf16 activations, S = 4096 + 256)
  zimage_swiglu   Z-Image FFN in-projection: silu(x Wg^T) * (x Wu^T), Q8_0 gate and
                  up [10240, 3840], bf16 [4352, 3840] (batch_matmul_swiglu_q8)
Weights are N(0, 0.02), activations N(0, 1), all from llmr_amd.synth streams.
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import gguf, synth

SEED = synth.BASE_SEED


@dataclasses.dataclass(frozen=True)
class Gemm:
    name: str
    M: int
    N: int
    K: int
    wtype: int
    xtype: int  # GGML type of the activations
    x_stream: int
    w_stream: int

    @property
    def flops(self) -> float:
        return 2.0 * self.M * self.N * self.K

    @property
    def bytes(self) -> int:
        """Algorithmic HBM bytes: packed weight + activations + f32 output."""
        xb = 4 if self.xtype == gguf.GGML_F32 else 2
        return self.N * gguf.row_bytes(self.wtype, self.K) + self.M * self.K * xb + self.M * self.N * 4


@dataclasses.dataclass(frozen=True)
class SwiGLU(Gemm):
    """Two GEMMs sharing the activations (gate weight from w_stream, up weight
    from w_stream + 1) and one f32 output."""

    @property
    def flops(self) -> float:
        return 4.0 * self.M * self.N * self.K

    @property
    def bytes(self) -> int:
        xb = 4 if self.xtype == gguf.GGML_F32 else 2
        return 2 * self.N * gguf.row_bytes(self.wtype, self.K) + self.M * self.K * xb + self.M * self.N * 4


@dataclasses.dataclass(frozen=True)
class Attention:
    name: str
    H: int
    S: int
    D: int
    n_txt: int
    grid_h: int
    grid_w: int
    axes: tuple
    theta: float

    @property
    def flops(self) -> float:
        return 4.0 * self.H * self.S * self.S * self.D

    @property
    def bytes(self) -> int:
        return 3 * self.H * self.S * self.D * 2 + self.S * self.H * self.D * 4


Q8_LINEAR = Gemm("q8_linear", 256, 3072, 3072, gguf.GGML_Q8_0, gguf.GGML_F32, 1, 2)
FLUX_ATTENTION = Attention("flux_attention", 24, 4608, 128, 512, 64, 64, (16, 56, 56), 10000.0)
FLUX_LINEAR1 = Gemm("flux_linear1", 4608, 21504, 3072, gguf.GGML_Q4_K, gguf.GGML_BF16, 6, 7)
FLUX_LINEAR2 = Gemm("flux_linear2", 4608, 3072, 15360, gguf.GGML_Q4_K, gguf.GGML_BF16, 8, 9)
FLUX_LINEAR1_F32 = Gemm("flux_linear1_f32", 4608, 21504, 3072, gguf.GGML_Q4_K, gguf.GGML_F32, 6, 7)
FLUX_LINEAR2_F32 = Gemm("flux_linear2_f32", 4608, 3072, 15360, gguf.GGML_Q4_K, gguf.GGML_F32, 8, 9)
ZIMAGE_QKV = Gemm("zimage_qkv", 4352, 11520, 3840, gguf.GGML_Q8_0, gguf.GGML_BF16, 10, 11)
ZIMAGE_O = Gemm("zimage_o", 4352, 3840, 3840, gguf.GGML_Q8_0, gguf.GGML_BF16, 12, 13)
ZIMAGE_DOWN = Gemm("zimage_down", 4352, 3840, 10240, gguf.GGML_Q8_0, gguf.GGML_BF16, 14, 15)
ZIMAGE_SWIGLU = SwiGLU("zimage_swiglu", 4352, 10240, 3840, gguf.GGML_Q8_0, gguf.GGML_BF16, 16, 17)
ZIMAGE_ATTENTION = Attention("zimage_attention", 30, 4352, 128, 256, 64, 64, (32, 48, 48), 256.0)

GEMMS = {g.name: g for g in (Q8_LINEAR, FLUX_LINEAR1, FLUX_LINEAR2, FLUX_LINEAR1_F32, FLUX_LINEAR2_F32, ZIMAGE_QKV,
                              ZIMAGE_O, ZIMAGE_DOWN)}
SWIGLUS = {g.name: g for g in (ZIMAGE_SWIGLU,)}


def gemm_weight_f32(g: Gemm) -> np.ndarray:
    return synth.normal(SEED, g.w_stream, g.N * g.K, 0.02).reshape(g.N, g.K)


def gemm_weight_blocks(g: Gemm) -> np.ndarray:
    return gguf.quantize(gemm_weight_f32(g), g.wtype)


def swiglu_up_blocks(g: SwiGLU) -> np.ndarray:
    """The up weight of a SwiGLU workload (gemm_weight_blocks gives the gate)."""
    w = synth.normal(SEED, g.w_stream + 1, g.N * g.K, 0.02).reshape(g.N, g.K)
    return gguf.quantize(w, g.wtype)


def gemm_activations_f32(g: Gemm) -> np.ndarray:
    """Activations as f32 values (already rounded to bf16 when xtype is BF16)."""
    x = synth.normal(SEED, g.x_stream, g.M * g.K).reshape(g.M, g.K)
    if g.xtype == gguf.GGML_BF16:
        x = round_bf16(x)
    elif g.xtype == gguf.GGML_F16:
        x = x.astype(np.float16).astype(np.float32)
    return x


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round f32 to the nearest bf16 (ties to even), returned as f32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).reshape(x.shape)


def attention_positions(a: Attention) -> np.ndarray:
    """Per-token axis positions [S, n_axes]: text tokens first with all-zero ids,
    then image tokens (0, row, col) (layout of precompute_flux_mrope,
    dependencies/flux.c3l/flux_dit.c3:410-445)."""
    pos = np.zeros((a.S, len(a.axes)), np.uint32)
    n_img = a.S - a.n_txt
    idx = np.arange(n_img)
    pos[a.n_txt:, 1] = idx // a.grid_w
    pos[a.n_txt:, 2] = idx % a.grid_w
    return pos


def rope_tables(pos: np.ndarray, axes, theta: float):
    """cos/sin [S, 64]: pair index runs over the axes; within an axis of dims
    a, pair k has freq = 1/theta^(2k/a) and angle = pos*freq, in f32
    (flux_dit.c3:447-486)."""
    S = pos.shape[0]
    cos_t = np.zeros((S, 64), np.float32)
    sin_t = np.zeros((S, 64), np.float32)
    pair = 0
    for ai, dims in enumerate(axes):
        k = np.arange(dims // 2, dtype=np.float32)
        freq = np.float32(1.0) / np.power(np.float32(theta), (2 * k) / np.float32(dims))
        ang = pos[:, ai].astype(np.float32)[:, None] * freq[None, :]
        cos_t[:, pair:pair + dims // 2] = np.cos(ang)
        sin_t[:, pair:pair + dims // 2] = np.sin(ang)
        pair += dims // 2
    return cos_t, sin_t


def rope_apply(x: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray) -> np.ndarray:
    """Interleaved-pair rotation on [H, S, 128] (mrope.slang:47-53)."""
    x0 = x[..., 0::2]
    x1 = x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * cos_t - x1 * sin_t
    out[..., 1::2] = x0 * sin_t + x1 * cos_t
    return out


def attention_inputs(a: Attention, heads=None):
    """Q, K, V as f16 [H, S, D] (RoPE on Q and K in f32, then one rounding).
    `heads` restricts generation to a (h0, h1) range of heads."""
    h0, h1 = heads if heads is not None else (0, a.H)
    n = a.S * a.D
    cos_t, sin_t = rope_tables(attention_positions(a), a.axes, a.theta)
    out = []
    for stream, rot in ((3, True), (4, True), (5, False)):
        x = synth.normal(SEED, stream, (h1 - h0) * n, start=h0 * n).reshape(h1 - h0, a.S, a.D)
        if rot:
            x = rope_apply(x, cos_t, sin_t)
        out.append(x.astype(np.float16))
    return tuple(out)
