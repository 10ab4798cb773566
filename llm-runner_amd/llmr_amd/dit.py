"""DiT blocks composed from the backend's entry points: the call sequences of
the reference's block functions, with its dispatch chains replaced by the
fused glue calls.

  ZImageBlock   dit_transformer_layer with adaLN
                (dependencies/zimage.c3l/dit.c3:1372-1627): RMSNorm + scale,
                QKV GEMM, head norm + RoPE + FA, O-proj, post-norm + tanh-gated
                residual, RMSNorm + scale, SwiGLU GEMM, down GEMM, post-norm +
                tanh-gated residual.
  FluxDiT       FluxDiTModel.forward (dependencies/flux.c3l/flux_dit.c3:1075-
                1210) over flux_dual_stream_block (:746-971) and
                flux_single_stream_block (:975-1071), at Flux.1-dev shapes:
                GELU (tanh) MLPs where the reference's Klein variant has SwiGLU
                halves, and per-block modulation projections where Klein shares
                one per block type.

Layout decisions (MI355X side, not the reference's):
  - the text and image streams live in one joint [n_txt + n_img, dim] f32
    residual buffer, text rows first (the reference's joint order), so the
    reference's stream concatenation and split copies (flux_dit.c3:1152-1153,
    880-887) disappear: each stream is a row range;
  - a fused weight is multiplied in one call over its full row range
    (Q | K | V, or Q | K | V | MLP-in for linear1) instead of one call per
    slot; the output columns are the slots side by side, exactly what the
    slot calls produce;
  - every GEMM and attention input is written by the glue in the activation
    type the kernels read (act_dtype, bf16 by default; Q/K/V in fp16).
"""
from __future__ import annotations

import dataclasses
import math

import torch

from . import capi, glue, workloads
from .gguf import GGML_Q4_K, GGML_Q8_0
from .ops import _TORCH_GGML, FlashAttentionPC, MatmulJob, NextImage, NextImages, QkvHeads, RenderGraph, Tensor, \
    build_next_images, default_graph, dispatch_batch_matmul, dispatch_batch_matmul_multi, \
    dispatch_batch_matmul_swiglu, dispatch_flash_attention, dispatch_flash_attention_rows, \
    split_swiglu_image_bytes, weight_image_bytes

HEAD_DIM = 128


def _qt(blocks: torch.Tensor, wtype: int, rows: int, cols: int) -> Tensor:
    return Tensor.quantized(blocks, wtype, rows, cols)


def _t(x: torch.Tensor) -> Tensor:
    return Tensor.from_torch(x)


# ---------------------------------------------------------------------------
# Z-Image block
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class ZImageLayerWeights:
    """The DiTLayerWeights a block reads (Q8_0 GEMM weights as raw blocks)."""
    wqkv: torch.Tensor      # [3*dim, dim]
    wo: torch.Tensor        # [dim, dim]
    w_gate: torch.Tensor    # [ffn, dim]
    w_up: torch.Tensor      # [ffn, dim]
    w_down: torch.Tensor    # [dim, ffn]
    attn_norm1: torch.Tensor  # f32 [dim]
    attn_norm2: torch.Tensor
    ffn_norm1: torch.Tensor
    ffn_norm2: torch.Tensor
    q_norm: torch.Tensor    # f32 [128]
    k_norm: torch.Tensor
    adaln: torch.Tensor     # f32 [4, dim]: scale_msa, gate_msa, scale_mlp, gate_mlp
    # w_gate's rows followed by w_up's in one buffer (w_gate and w_up are then
    # views of it; a loader concatenates the two tensors' blocks once), or None
    w_gate_up: torch.Tensor | None = None


class ZImageBlock:
    """One Z-Image transformer layer with adaLN, on preallocated buffers for a
    fixed (dim, n_heads, ffn_dim, seq_len). The per-layer adaLN projection of
    the timestep embedding (an M=1 linear_proj, dit.c3:1398-1417) is an input
    here: `weights.adaln` holds its four chunks."""

    EPS = 1e-5  # batch_rmsnorm and batch_head_norm eps (dit.c3:1423, 1447)

    def __init__(self, dim: int, n_heads: int, ffn_dim: int, seq_len: int, act_dtype=torch.bfloat16,
                 device="cuda", g: RenderGraph | None = None, images_ahead: bool = True):
        if dim != n_heads * HEAD_DIM:
            raise ValueError("dim must be n_heads * 128")
        self.dim, self.n_heads, self.ffn, self.S = dim, n_heads, ffn_dim, seq_len
        self.g = g or default_graph()
        S = seq_len
        e = dict(device=device)
        # the block's four GEMMs (QKV, O-proj, gate | up SwiGLU, down) as an
        # image chain when they run two-pass: each call builds the next one's
        # weight images (the SwiGLU's idle workgroups the down projection's)
        self.ahead = None
        if images_ahead and S >= TWO_PASS_MIN_TOKENS and dim % 64 == 0 and ffn_dim % 64 == 0 and \
                act_dtype in (torch.float16, torch.bfloat16):
            cus = torch.cuda.get_device_properties(torch.device(device)).multi_processor_count
            self.ahead = _ImageChain([([None], 3 * dim, dim, (S,)), ([None], dim, dim, (S,)),
                                      ([None], 2 * ffn_dim, dim, (S,), 0), ([None], dim, ffn_dim, (S,))],
                                     _TORCH_GGML[act_dtype], device, cus, GGML_Q8_0)
        self.xa = torch.empty(S, dim, dtype=act_dtype, **e)          # GEMM inputs of width dim
        self.q = torch.empty(n_heads, S, HEAD_DIM, dtype=torch.float16, **e)
        self.k = torch.empty_like(self.q)
        self.v = torch.empty_like(self.q)
        self.t = torch.empty(S, dim, dtype=torch.float32, **e)      # O-proj / down outputs
        self.f = torch.empty(S, ffn_dim, dtype=torch.float32, **e)  # SwiGLU output
        self.fa = torch.empty(S, ffn_dim, dtype=act_dtype, **e)     # down-projection input

    def forward(self, w: ZImageLayerWeights, hidden: torch.Tensor, rope_cos: torch.Tensor,
                rope_sin: torch.Tensor) -> torch.Tensor:
        """hidden f32 [seq_len, dim], updated in place (and returned)."""
        g, S, dim, H, ffn, eps = self.g, self.S, self.dim, self.n_heads, self.ffn, self.EPS
        if hidden.shape != (S, dim) or hidden.dtype != torch.float32:
            raise ValueError("hidden must be f32 [seq_len, dim]")
        ch = self.ahead if w.w_gate_up is not None else None
        wqkv, wo = _qt(w.wqkv, GGML_Q8_0, 3 * dim, dim), _qt(w.wo, GGML_Q8_0, dim, dim)
        wdown = _qt(w.w_down, GGML_Q8_0, dim, ffn)
        if ch is not None:
            wgu = _qt(w.w_gate_up, GGML_Q8_0, 2 * ffn, dim)
            ch.bind([[wqkv], [wo], [wgu], [wdown]])
            ch.start(g)

        def mm(jobs, N, K, epilogue=capi.EPI_STORE, split=0, heads=None):
            if ch is None:
                if epilogue == capi.EPI_STORE and heads is None:  # the plain projections
                    j = jobs[0]
                    dispatch_batch_matmul(g, j.weight, j.input, _t(j.output), N, K, j.seq_len, 0)
                else:
                    dispatch_batch_matmul_multi(g, jobs, N, K, epilogue, split, heads=heads)
                return
            images, nxt = ch.take(jobs, N, K)
            dispatch_batch_matmul_multi(g, jobs, N, K, epilogue, split, images=images, next_images=nxt,
                                        heads=heads)
        try:
            return self._forward(w, hidden, rope_cos, rope_sin, wqkv, wo, wdown, mm)
        finally:
            if ch is not None:  # a failed forward leaves no chain half-taken
                ch.active = False

    def _forward(self, w, hidden, rope_cos, rope_sin, wqkv, wo, wdown, mm):
        g, S, dim, H, ffn, eps = self.g, self.S, self.dim, self.n_heads, self.ffn, self.EPS
        # A: pre-attention RMSNorm, * (1 + scale_msa)                 (dit.c3:1421-1432)
        glue.batch_rmsnorm(hidden, w.attn_norm1, self.xa, eps, mod_scale=w.adaln[0], g=g)
        # B, C: Q | K | V in one call over the fused weight, with the head
        # norm, RoPE and head-major fp16 Q/K/V done on its result
        # (dit.c3:1435-1473); attention                               (dit.c3:1476-1483)
        mm([MatmulJob(wqkv, _t(self.xa), None, S)], 3 * dim, dim,
           heads=QkvHeads(self.q, self.k, self.v, H, [(w.q_norm, w.k_norm, 0)], eps, (rope_cos, rope_sin)))
        # (the attention rows go straight into the O-proj input, rounded to the
        # activation type: the reference's attention output plus its copy)
        dispatch_flash_attention_rows(g, _t(self.q), _t(self.k), _t(self.v), self.xa,
                                      FlashAttentionPC(HEAD_DIM, H, S, 1.0 / math.sqrt(HEAD_DIM)))
        # D: O-proj; hidden += tanh(gate_msa) * rmsnorm(o-proj)        (dit.c3:1488-1503)
        mm([MatmulJob(wo, _t(self.xa), self.t, S)], dim, dim)
        # E: FFN pre-norm, * (1 + scale_mlp), in the same pass         (dit.c3:1545-1554)
        if dim <= 4096:
            glue.gated_residual_rmsnorm(hidden, self.t, w.adaln[1], capi.GATE_TANH, w.attn_norm2, eps, w.ffn_norm1,
                                        self.xa, eps, mod_scale=w.adaln[2], g=g)
        else:
            glue.gated_residual(hidden, self.t, w.adaln[1], capi.GATE_TANH, w.attn_norm2, eps, g=g)
            glue.batch_rmsnorm(hidden, w.ffn_norm1, self.xa, eps, mod_scale=w.adaln[2], g=g)
        # F: SwiGLU in-projection, down-projection                     (dit.c3:1562-1596)
        if w.w_gate_up is not None:
            # gate | up in one weight: silu(gate) * up straight into the
            # down-projection input in the activation type (the split-SwiGLU
            # epilogue with no plain columns); on the two-pass kernel bit for
            # bit the SwiGLU's f32 output and its copy below
            mm([MatmulJob(_qt(w.w_gate_up, GGML_Q8_0, 2 * ffn, dim), _t(self.xa), None, S, 0, None, self.fa)],
               2 * ffn, dim, capi.EPI_SPLIT_SWIGLU, 0)
        else:
            dispatch_batch_matmul_swiglu(g, _qt(w.w_gate, GGML_Q8_0, ffn, dim), _qt(w.w_up, GGML_Q8_0, ffn, dim),
                                         _t(self.xa), _t(self.f), ffn, dim, S)
            glue.activation(self.f, self.fa, capi.ACT_COPY, g=g)
        mm([MatmulJob(wdown, _t(self.fa), self.t, S)], dim, ffn)
        # G: hidden += tanh(gate_mlp) * rmsnorm(down)                  (dit.c3:1600-1610)
        glue.gated_residual(hidden, self.t, w.adaln[3], capi.GATE_TANH, w.ffn_norm2, eps, g=g)
        return hidden


def zimage_layer_weights(dim: int, n_heads: int, ffn: int, device="cuda", seed: int = workloads.SEED,
                         base_stream: int = 10) -> ZImageLayerWeights:
    """Synthetic Z-Image layer weights: Q8_0 GEMM weights ~N(0, 0.02) quantized
    on the host (the same streams as the zimage_* GEMM workloads when the
    shapes are the full block's), norm weights 1 + N(0, 0.1), adaLN chunks
    N(0, 0.5)."""
    from . import gguf, synth

    def q8(rows, cols, stream):
        w = synth.normal(seed, stream, rows * cols, 0.02).reshape(rows, cols)
        return torch.from_numpy(gguf.quantize(w, GGML_Q8_0)).to(device)

    def vec(n, stream, mean, std):
        return torch.from_numpy(mean + synth.normal(seed, stream, n, std)).to(device)

    b = base_stream
    gate_up = torch.cat([q8(ffn, dim, b + 6), q8(ffn, dim, b + 7)])  # gate rows, then up rows
    half = gate_up.numel() // 2
    return ZImageLayerWeights(
        wqkv=q8(3 * dim, dim, b + 1), wo=q8(dim, dim, b + 3), w_gate=gate_up[:half], w_up=gate_up[half:],
        w_down=q8(dim, ffn, b + 5),
        attn_norm1=vec(dim, b + 20, 1.0, 0.1), attn_norm2=vec(dim, b + 21, 1.0, 0.1),
        ffn_norm1=vec(dim, b + 22, 1.0, 0.1), ffn_norm2=vec(dim, b + 23, 1.0, 0.1),
        q_norm=vec(HEAD_DIM, b + 24, 1.0, 0.1), k_norm=vec(HEAD_DIM, b + 25, 1.0, 0.1),
        adaln=vec(4 * dim, b + 26, 0.0, 0.5).reshape(4, dim), w_gate_up=gate_up)


# ---------------------------------------------------------------------------
# Flux (Flux.1-dev shapes)
# ---------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class FluxConfig:
    dim: int = 3072
    n_heads: int = 24
    mlp: int = 12288
    n_double: int = 19
    n_single: int = 38
    text_dim: int = 4096
    n_txt: int = 512
    latent_ch: int = 16
    latent_h: int = 128
    latent_w: int = 128
    patch: int = 2
    t_emb_dim: int = 256
    axes: tuple = (16, 56, 56)
    theta: float = 10000.0
    # "gelu": the Flux.1-dev MLP (in-projection [mlp, dim], GELU); "swiglu":
    # the reference's own Flux.2 MLP (in-projection [2 mlp, dim]: gate rows,
    # then up rows; silu(gate) * up, flux_dit.c3:917-931, 1013-1018, 1049-1055)
    mlp_act: str = "gelu"

    @property
    def mlp_in(self) -> int:
        """Rows of a block's MLP in-projection (and of linear1 past 3 dim)."""
        return 2 * self.mlp if self.mlp_act == "swiglu" else self.mlp

    @property
    def patch_dim(self) -> int:
        return self.latent_ch * self.patch * self.patch

    @property
    def n_img(self) -> int:
        return (self.latent_h // self.patch) * (self.latent_w // self.patch)

    @property
    def seq(self) -> int:
        return self.n_txt + self.n_img

    def gemm_flops(self) -> float:
        """2MNK over every token-wise GEMM plus 4*H*S^2*D per attention (the
        modulation and timestep projections, M = 1, are not counted)."""
        d, m, mi, ni, nt, S = self.dim, self.mlp, self.mlp_in, self.n_img, self.n_txt, self.seq
        per_stream = 3 * d * d + d * d + mi * d + d * m
        double = 2.0 * (ni + nt) * per_stream + 4.0 * self.n_heads * S * S * HEAD_DIM
        single = 2.0 * S * ((3 * d + mi) * d + d * (d + m)) + 4.0 * self.n_heads * S * S * HEAD_DIM
        io = 2.0 * ni * self.patch_dim * d + 2.0 * nt * self.text_dim * d + 2.0 * ni * d * self.patch_dim
        return self.n_double * double + self.n_single * single + io


FLUX_DEV = FluxConfig()


@dataclasses.dataclass
class FluxDoubleWeights:
    img_mod: torch.Tensor   # Q4_K [6*dim, dim]
    txt_mod: torch.Tensor
    img_qkv: torch.Tensor   # Q4_K [3*dim, dim]
    txt_qkv: torch.Tensor
    img_proj: torch.Tensor  # Q4_K [dim, dim]
    txt_proj: torch.Tensor
    img_mlp0: torch.Tensor  # Q4_K [mlp, dim] (swiglu: [2 mlp, dim], gate rows then up rows)
    txt_mlp0: torch.Tensor
    img_mlp2: torch.Tensor  # Q4_K [dim, mlp]
    txt_mlp2: torch.Tensor
    img_q_norm: torch.Tensor  # f32 [128]
    img_k_norm: torch.Tensor
    txt_q_norm: torch.Tensor
    txt_k_norm: torch.Tensor


@dataclasses.dataclass
class FluxSingleWeights:
    mod: torch.Tensor       # Q4_K [3*dim, dim]
    linear1: torch.Tensor   # Q4_K [3*dim + mlp, dim] (swiglu: [3*dim + 2 mlp, dim])
    linear2: torch.Tensor   # Q4_K [dim, dim + mlp]
    q_norm: torch.Tensor
    k_norm: torch.Tensor


@dataclasses.dataclass
class FluxGlobalWeights:
    img_in: torch.Tensor      # Q8_0 [dim, patch_dim] (patch_dim = 64 is not a Q4_K row)
    txt_in: torch.Tensor      # Q4_K [dim, text_dim]
    time_in0: torch.Tensor    # Q4_K [dim, t_emb_dim]
    time_in1: torch.Tensor    # Q4_K [dim, dim]
    final_mod: torch.Tensor   # Q4_K [2*dim, dim]
    final_linear: torch.Tensor  # Q4_K [patch_dim, dim]


def flux_weights(cfg: FluxConfig, device="cuda", seed: int = workloads.SEED, g: RenderGraph | None = None):
    """Random-init Flux weights: Q4_K tensors ~N(0, 0.02) generated and
    quantized on the device (llmr_synth_q4k), one stream per tensor; norm
    weights 1 + N(0, 0.1); img_in Q8_0 quantized on the host."""
    from . import gguf, synth
    g = g or default_graph()
    d, m = cfg.dim, cfg.mlp
    counter = [1000]

    def q4(rows, cols):
        counter[0] += 1
        return glue.synth_q4k(rows, cols, counter[0], 0.02, seed, device, g)

    def norm():
        counter[0] += 1
        return torch.from_numpy(1.0 + synth.normal(seed, counter[0], HEAD_DIM, 0.1)).to(device)

    mi = cfg.mlp_in
    doubles = [FluxDoubleWeights(q4(6 * d, d), q4(6 * d, d), q4(3 * d, d), q4(3 * d, d), q4(d, d), q4(d, d),
                                 q4(mi, d), q4(mi, d), q4(d, m), q4(d, m), norm(), norm(), norm(), norm())
               for _ in range(cfg.n_double)]
    singles = [FluxSingleWeights(q4(3 * d, d), q4(3 * d + mi, d), q4(d, d + m), norm(), norm())
               for _ in range(cfg.n_single)]
    w_in = synth.normal(seed, 999, d * cfg.patch_dim, 0.02).reshape(d, cfg.patch_dim)
    glob = FluxGlobalWeights(torch.from_numpy(gguf.quantize(w_in, GGML_Q8_0)).to(device), q4(d, cfg.text_dim),
                             q4(d, cfg.t_emb_dim), q4(d, d), q4(2 * d, d), q4(cfg.patch_dim, d))
    return glob, doubles, singles


# Checkpoint tensor names: the BFL Flux.1-dev layout this model uses (per-block
# img_mod / txt_mod / modulation weights, a GELU MLP with img_mlp.0 of
# [mlp, dim], linear1 of [3 dim + mlp, dim]; with mlp_act "swiglu" the same
# names hold the SwiGLU halves, img_mlp.0 of [2 mlp, dim] and linear1 of
# [3 dim + 2 mlp, dim]). The reference's loader (load_flux_dit,
# flux_dit.c3:664-744) reads the Flux Klein layout: the SwiGLU halves, and
# shared double_stream_modulation_img/txt and single_stream_modulation
# weights instead of per-block ones, so its checkpoints do not load here
# unchanged.
_FLUX_GLOBAL = {"img_in": "img_in.weight", "txt_in": "txt_in.weight", "time_in0": "time_in.in_layer.weight",
                "time_in1": "time_in.out_layer.weight", "final_mod": "final_layer.adaLN_modulation.1.weight",
                "final_linear": "final_layer.linear.weight"}
_FLUX_DOUBLE = {"img_mod": "img_mod.lin.weight", "txt_mod": "txt_mod.lin.weight",
                "img_qkv": "img_attn.qkv.weight", "txt_qkv": "txt_attn.qkv.weight",
                "img_proj": "img_attn.proj.weight", "txt_proj": "txt_attn.proj.weight",
                "img_mlp0": "img_mlp.0.weight", "txt_mlp0": "txt_mlp.0.weight",
                "img_mlp2": "img_mlp.2.weight", "txt_mlp2": "txt_mlp.2.weight",
                "img_q_norm": "img_attn.norm.query_norm.scale", "img_k_norm": "img_attn.norm.key_norm.scale",
                "txt_q_norm": "txt_attn.norm.query_norm.scale", "txt_k_norm": "txt_attn.norm.key_norm.scale"}
_FLUX_SINGLE = {"mod": "modulation.lin.weight", "linear1": "linear1.weight", "linear2": "linear2.weight",
                "q_norm": "norm.query_norm.scale", "k_norm": "norm.key_norm.scale"}


def _flux_shapes(cfg: FluxConfig):
    d, m, mi = cfg.dim, cfg.mlp, cfg.mlp_in
    glob = {"img_in": (d, cfg.patch_dim), "txt_in": (d, cfg.text_dim), "time_in0": (d, cfg.t_emb_dim),
            "time_in1": (d, d), "final_mod": (2 * d, d), "final_linear": (cfg.patch_dim, d)}
    dbl = {"img_mod": (6 * d, d), "txt_mod": (6 * d, d), "img_qkv": (3 * d, d), "txt_qkv": (3 * d, d),
           "img_proj": (d, d), "txt_proj": (d, d), "img_mlp0": (mi, d), "txt_mlp0": (mi, d),
           "img_mlp2": (d, m), "txt_mlp2": (d, m)}
    sgl = {"mod": (3 * d, d), "linear1": (3 * d + mi, d), "linear2": (d, d + m)}
    return glob, dbl, sgl


def save_flux_gguf(path: str, cfg: FluxConfig, glob: FluxGlobalWeights, doubles, singles) -> int:
    """Writes Flux weights (device tensors) as a GGUF checkpoint with the
    BFL Flux.1-dev tensor names and shapes (not the Klein layout the
    reference loads): matrices in their quantized blocks (img_in Q8_0, the
    rest Q4_K), norm scales F32. Returns the file size."""
    from . import gguf_file
    gs, ds, ss = _flux_shapes(cfg)
    ents = []

    def add(name, t, shape, gtype):
        data = t.detach().cpu().numpy()
        ents.append(gguf_file.TensorEntry(name, gtype, shape, data.tobytes()))

    for k, name in _FLUX_GLOBAL.items():
        add(name, getattr(glob, k), gs[k], GGML_Q8_0 if k == "img_in" else GGML_Q4_K)
    for i, w in enumerate(doubles):
        for k, name in _FLUX_DOUBLE.items():
            t = getattr(w, k)
            if k in ds:
                add(f"double_blocks.{i}.{name}", t, ds[k], GGML_Q4_K)
            else:
                add(f"double_blocks.{i}.{name}", t.float(), (HEAD_DIM,), 0)
    for i, w in enumerate(singles):
        for k, name in _FLUX_SINGLE.items():
            t = getattr(w, k)
            if k in ss:
                add(f"single_blocks.{i}.{name}", t, ss[k], GGML_Q4_K)
            else:
                add(f"single_blocks.{i}.{name}", t.float(), (HEAD_DIM,), 0)
    meta = {"general.architecture": "flux", "flux.dim": cfg.dim, "flux.heads": cfg.n_heads, "flux.mlp": cfg.mlp,
            "flux.double_blocks": cfg.n_double, "flux.single_blocks": cfg.n_single}
    return gguf_file.write_gguf(path, ents, meta)


def flux_weights_from_gguf(path: str, cfg: FluxConfig, device="cuda"):
    """Flux.1-dev weights loaded from a GGUF checkpoint in the layout of
    save_flux_gguf, the way load_flux_dit (flux_dit.c3:664-744) loads its
    Klein checkpoints: every matrix uploaded unchanged through the native
    parser (upload_weight), norm scales widened to f32. Shapes and types are
    checked against cfg (the GEMMs take Q4_K and Q8_0)."""
    from . import gguf_file
    gs, ds, ss = _flux_shapes(cfg)
    with gguf_file.GGUFFile(path) as f:
        def mat(name, shape):
            t = f.by_name.get(name)
            if t is None:
                raise KeyError(f"{path}: no tensor {name}")
            if t.shape != tuple(shape) or t.ggml_type not in (GGML_Q8_0, GGML_Q4_K):
                raise ValueError(f"{name}: {t.shape} of type {t.ggml_type}, expected {shape} in Q8_0/Q4_K")
            return f.upload(name, device)

        def norm(name):
            if name not in f.by_name:
                raise KeyError(f"{path}: no tensor {name}")
            return f.upload_f32(name, device).reshape(-1)

        glob = FluxGlobalWeights(**{k: mat(n, gs[k]) for k, n in _FLUX_GLOBAL.items()})
        doubles = [FluxDoubleWeights(**{k: (mat(f"double_blocks.{i}.{n}", ds[k]) if k in ds
                                            else norm(f"double_blocks.{i}.{n}"))
                                        for k, n in _FLUX_DOUBLE.items()}) for i in range(cfg.n_double)]
        singles = [FluxSingleWeights(**{k: (mat(f"single_blocks.{i}.{n}", ss[k]) if k in ss
                                            else norm(f"single_blocks.{i}.{n}"))
                                        for k, n in _FLUX_SINGLE.items()}) for i in range(cfg.n_single)]
    return glob, doubles, singles


def flux_rope(cfg: FluxConfig, device="cuda"):
    """cos/sin [seq, 64] for text ids (0,0,0) then image ids (0, row, col)
    (precompute_flux_mrope, flux_dit.c3:396-529), computed on the host."""
    att = workloads.Attention("flux", cfg.n_heads, cfg.seq, HEAD_DIM, cfg.n_txt, cfg.latent_h // cfg.patch,
                              cfg.latent_w // cfg.patch, cfg.axes, cfg.theta)
    cos_t, sin_t = workloads.rope_tables(workloads.attention_positions(att), cfg.axes, cfg.theta)
    return torch.from_numpy(cos_t).to(device), torch.from_numpy(sin_t).to(device)


# Token count from which a GEMM runs two-pass (a 16-bit weight image, then
# the matrix-core pass); the C-ABI makes the same choice.
TWO_PASS_MIN_TOKENS = 2048


class _ImageChain:
    """Weight images of a fixed sequence of GEMM groups (one multi launch
    each: one or two Q4_K/Q8_0 weights of one shape N x K, rows from 0, the
    token counts of its jobs and, for a SPLIT_SWIGLU group, its split (a
    weight's image then the plain image of its first split rows followed by
    the SwiGLU image of its (N - split) / 2 outputs: two images), built
    ahead. Call k builds what is left of group k + 1's images (its GEMM's
    idle workgroups, those without a tile in its last round, as far as they
    reach, the rest right after it), then, while its idle room lasts, parts
    of group k + 2's and k + 3's images in order: whole 256-row panels (128
    outputs of a SwiGLU image) of one image, a next image each (at most
    eight a call). The first group's images are built before it. Four
    buffers rotate (group k in buffer k % 4: at most three groups are built
    ahead of the one running, none into the buffer it reads). The room is
    estimated here from the launch's tile count; a wrong estimate only moves
    items into the image launch after the GEMM. The results are those of
    dispatch_batch_matmul_multi without images, bit for bit. A group's
    weights may be None at construction (the shapes alone plan the chain);
    bind() then sets them before start()."""

    NBUF = 4        # buffers (groups built ahead: NBUF - 1)
    MAX_PARTS = 8   # next images a call takes

    def __init__(self, groups, input_dtype: int, device, cus: int, wtype: int = GGML_Q4_K):
        if any(self._entries(gr) > self.MAX_PARTS for gr in groups):
            raise ValueError("a group's images must fit one call's next images")
        self.groups, self.xtype = list(groups), input_dtype
        per = max(len(gr[0]) * self._image_bytes(gr) for gr in groups)
        self.bufs = [torch.empty(per, dtype=torch.uint8, device=device) for _ in range(self.NBUF)]
        self.builds = self.plan(groups, cus, wtype)  # call k -> the (group, image, p0, p1) parts it builds
        self.bound = False
        if all(w is not None for gr in groups for w in gr[0]):
            self.bind([gr[0] for gr in groups])
        self.k = 0
        self.active = False  # between start() and the last group's take()

    def bind(self, weights) -> None:
        """The weights of each group (a list per group, as many as planned)."""
        if len(weights) != len(self.groups) or any(len(w) != len(gr[0]) for w, gr in zip(weights, self.groups)):
            raise ValueError("one weight list per group, as many weights as planned")
        self.groups = [(list(w),) + tuple(gr[1:]) for w, gr in zip(weights, self.groups)]
        self.nexts = [self._parts(c) for c in range(len(self.groups))]  # call c's NextImages (or None)
        self.bound = True

    @classmethod
    def plan(cls, groups, cus: int, wtype: int = GGML_Q4_K):
        """For each call c, the image parts (group j, image e, panels [p0, p1))
        it builds, in order: what is left of group c + 1's images, then parts
        of group c + 2's and c + 3's images in order while whole panels fit
        in what is left of the call's room and a next image is left."""
        n = len(groups)
        builds = [[] for _ in range(n)]
        done = [[0] * cls._entries(gr) for gr in groups]  # panels of each image assigned so far
        for c in range(n - 1):
            room, slots = cls._room(groups[c], cus, wtype), cls.MAX_PARTS
            later = False
            for j in range(c + 1, min(n, c + cls.NBUF)):
                ents = cls._entry_panels(groups[j])
                per = cls._stage_groups(groups[j])  # items of one panel
                for e, panels in enumerate(ents):
                    p0 = done[j][e]
                    if p0 == panels:
                        continue
                    if j == c + 1:  # the next group: all of what is left
                        p1 = panels
                    else:
                        if not later:  # a margin for the groups after next
                            room = room * 3 // 4
                            later = True
                        if slots == 0 or room < per:
                            break
                        p1 = min(panels, p0 + room // per)
                    builds[c].append((j, e, p0, p1))
                    room -= (p1 - p0) * per
                    slots -= 1
                    done[j][e] = p1
                    if p1 < panels:  # the room ran out inside this image
                        break
                else:
                    continue
                break
        return builds

    @staticmethod
    def _split(group):
        return group[4] if len(group) > 4 else None

    @staticmethod
    def _stage_groups(group) -> int:
        """Items of one panel: its K stages in groups of four."""
        return -(-(group[2] // 64) // 4)

    @classmethod
    def _entry_panels(cls, group) -> list:
        """Panels of the group's images in order: one image per weight; a split
        SwiGLU weight's plain rows (256 a panel, when split > 0), then its
        SwiGLU rows (128 outputs a panel)."""
        ws, N = group[0], group[1]
        split = cls._split(group)
        if split is None:
            return [-(-N // 256)] * len(ws)
        one = ([split // 256] if split else []) + [-(-((N - split) // 2) // 128)]
        return one * len(ws)

    @classmethod
    def _entry_items(cls, group) -> list:
        """Image items ((panel, 4 K stages) each) of the group's images."""
        per = cls._stage_groups(group)
        return [p * per for p in cls._entry_panels(group)]

    @classmethod
    def _entries(cls, group) -> int:
        """Images of a group."""
        return len(cls._entry_panels(group))

    @classmethod
    def _panels(cls, group) -> int:
        """Panels of one weight's image, also the GEMM's column tiles."""
        return sum(cls._entry_panels(group)) // len(group[0])

    @classmethod
    def _image_bytes(cls, group) -> int:
        ws, N, K = group[:3]
        split = cls._split(group)
        return weight_image_bytes(N, K) if split is None else split_swiglu_image_bytes(split, (N - split) // 2, K)

    @classmethod
    def _items(cls, group) -> int:
        """Image items of a group: (256-row panel, 4 K stages) each."""
        return sum(cls._entry_items(group))

    @classmethod
    def _room(cls, group, cus: int, wtype: int = GGML_Q4_K) -> int:
        """Items of weight type wtype the group's GEMM can build on its
        workgroups without a tile in the last round: one per four of its K
        stages each (Q8_0: per eight)."""
        K, Ms = group[2], group[3]
        tiles = sum(-(-M // 256) for M in Ms) * cls._panels(group)
        rem = tiles % cus
        return 0 if rem == 0 else (cus - rem) * max(1, K // (512 if wtype == GGML_Q8_0 else 256))

    def _views(self, k: int):
        n = self._image_bytes(self.groups[k])
        return [self.bufs[k % self.NBUF][i * n:(i + 1) * n] for i in range(len(self.groups[k][0]))]

    def _part(self, j: int, e: int, p0: int, p1: int) -> NextImage:
        """Panels [p0, p1) of group j's image e as a next image."""
        gr = self.groups[j]
        ws, N, K = gr[:3]
        split = self._split(gr)
        per_w = 1 if split is None or split == 0 else 2  # images per weight
        w, kind = divmod(e, per_w)
        view = self._views(j)[w]
        panel = weight_image_bytes(256, K)  # bytes of one panel (either arrangement)
        if split is None or (split and kind == 0):  # plain rows
            rows = N if split is None else split
            n = min(256 * p1, rows) - 256 * p0
            return NextImage(ws[w], n, K, view[p0 * panel:p1 * panel], 256 * p0)
        f = (N - split) // 2
        base = weight_image_bytes(split, K) if split else 0
        n = min(128 * p1, f) - 128 * p0
        return NextImage(ws[w], n, K, view[base + p0 * panel:base + p1 * panel], split + 128 * p0, True, f)

    def _parts(self, c: int):
        if not self.builds[c]:
            return None
        return NextImages([self._part(j, e, p0, p1) for j, e, p0, p1 in self.builds[c]])

    def start(self, g: RenderGraph) -> None:
        """Before the first group: its images."""
        if not self.bound:
            raise RuntimeError("weight-image chain started before its weights were bound")
        self.k = 0
        self.active = True
        gr = self.groups[0]
        build_next_images(g, NextImages([self._part(0, e, 0, p) for e, p in enumerate(self._entry_panels(gr))]),
                          self.xtype)

    def take(self, jobs, N: int, K: int):
        """(images, next_images) for the next group's call, whose jobs must be
        that group's GEMMs (the same weights, in order, and shape): images are
        matched to jobs by position, which the C-ABI cannot check."""
        k = self.k
        ws, gN, gK = self.groups[k][:3]
        if (gN, gK) != (N, K) or [w.ptr() for w in ws] != [j.weight.ptr() for j in jobs]:
            self.active = False
            raise RuntimeError(f"weight-image chain out of step: group {k} holds other weights than this call's")
        self.k += 1
        self.active = self.k < len(self.groups)
        return self._views(k), self.nexts[k]


class FluxDiT:
    """One denoising forward of a Flux-shaped DiT on preallocated buffers."""

    LN_EPS = 1e-6   # batch_layernorm eps (flux_dit.c3:766)
    HN_EPS = 1e-6   # batch_head_norm eps (flux_dit.c3:813)

    def __init__(self, cfg: FluxConfig, glob: FluxGlobalWeights, doubles, singles, act_dtype=torch.bfloat16,
                 device="cuda", g: RenderGraph | None = None, images_ahead: bool = True):
        self.cfg, self.glob, self.doubles, self.singles = cfg, glob, doubles, singles
        self.g = g or default_graph()
        c, e = cfg, dict(device=device)
        S, d, m, nt = c.seq, c.dim, c.mlp, c.n_txt
        # the blocks' GEMM groups in issue order, each group's weight images
        # built by the call before it (when the GEMMs run two-pass); the
        # SwiGLU form's in-projections are SPLIT_SWIGLU groups (plain rows,
        # then SwiGLU-arranged gate / up rows)
        self.ahead = None
        if images_ahead and S >= TWO_PASS_MIN_TOKENS and d % 64 == 0 and m % 64 == 0 and \
                act_dtype in (torch.float16, torch.bfloat16):
            def q4(t, K):
                return _qt(t, GGML_Q4_K, t.numel() // (K // 256 * 144), K)
            sw = cfg.mlp_act == "swiglu"
            rows, sp0, sp1 = (2 * m, (0,), (3 * d,)) if sw else (m, (), ())  # MLP-in rows, splits
            groups = []
            two = (nt, S - nt)  # a double block's text and image jobs
            for w in doubles:
                groups += [([q4(w.txt_qkv, d), q4(w.img_qkv, d)], 3 * d, d, two),
                           ([q4(w.txt_proj, d), q4(w.img_proj, d)], d, d, two),
                           ([q4(w.txt_mlp0, d), q4(w.img_mlp0, d)], rows, d, two) + sp0,
                           ([q4(w.txt_mlp2, m), q4(w.img_mlp2, m)], d, m, two)]
            for w in singles:
                groups += [([q4(w.linear1, d)], 3 * d + rows, d, (S,)) + sp1,
                           ([q4(w.linear2, d + m)], d, d + m, (S,))]
            if groups:
                cus = torch.cuda.get_device_properties(torch.device(device)).multi_processor_count
                self.ahead = _ImageChain(groups, _TORCH_GGML[act_dtype], device, cus)
        self.rope = flux_rope(cfg, device)
        self.hidden = torch.empty(S, d, dtype=torch.float32, **e)   # joint residual stream, text rows first
        self.xa = torch.empty(S, d, dtype=act_dtype, **e)             # GEMM inputs of width dim
        self.patches = torch.empty(c.n_img, c.patch_dim, dtype=act_dtype, **e)
        self.q = torch.empty(c.n_heads, S, HEAD_DIM, dtype=torch.float16, **e)
        self.k = torch.empty_like(self.q)
        self.v = torch.empty_like(self.q)
        self.o = torch.empty(S, d, dtype=torch.float32, **e)
        self.cat = torch.empty(S, d + m, dtype=act_dtype, **e)  # linear2 input [attention | gelu(MLP)]
        # the double block's MLP activations [S, mlp] (dense: a GEMM input)
        # share the single block's concat buffer; the block types never overlap
        self.fa = self.cat.view(-1)[:S * m].view(S, m)
        self.t_emb = torch.empty(1, c.t_emb_dim, dtype=torch.float32, **e)
        self.vec0 = torch.empty(1, d, dtype=torch.float32, **e)
        self.vec = torch.empty(1, d, dtype=torch.float32, **e)
        n_mod = (12 * c.n_double + 3 * c.n_single + 2) * d
        self.mods = torch.empty(1, n_mod, dtype=torch.float32, **e)
        self.velocity = torch.empty(c.n_img, c.patch_dim, dtype=torch.float32, **e)
        self.out = torch.empty(c.latent_ch, c.latent_h, c.latent_w, dtype=torch.float32, **e)

    # GEMM helper: rows [r0, r0+M) of x (activation type) times weight -> rows of y (f32)
    def _mm(self, w: torch.Tensor, wtype: int, N: int, K: int, x: torch.Tensor, y: torch.Tensor) -> None:
        dispatch_batch_matmul(self.g, _qt(w, wtype, N, K), _t(x), _t(y), N, K, x.shape[0], 0)

    def _mod(self, i: int, n: int) -> torch.Tensor:
        d = self.cfg.dim
        return self.mods[0, i * d:(i + n) * d].view(n, d)

    def forward(self, latent: torch.Tensor, txt: torch.Tensor, sigma: float) -> torch.Tensor:
        """latent f32 [C, H, W], txt [n_txt, text_dim] (activation type) ->
        velocity f32 [C, H, W] (self.out)."""
        c, g = self.cfg, self.g
        d, nt = c.dim, c.n_txt
        S = c.seq
        hid_t, hid_i = self.hidden[:nt], self.hidden[nt:]
        # 1-3: patchify; img_in and txt_in straight into the joint stream (flux_dit.c3:1093-1114)
        glue.patchify(latent, self.patches, c.patch, g=g)
        self._mm(self.glob.img_in, GGML_Q8_0, d, c.patch_dim, self.patches, hid_i)
        self._mm(self.glob.txt_in, GGML_Q4_K, d, c.text_dim, txt, hid_t)
        # 4: timestep embedding (sigma * 1000) -> MLP (flux_dit.c3:1121-1129)
        glue.timestep_embed(self.t_emb, sigma * 1000.0, g=g)
        self._mm(self.glob.time_in0, GGML_Q4_K, d, c.t_emb_dim, self.t_emb, self.vec0)
        glue.activation(self.vec0, self.vec0, capi.ACT_SILU, g=g)
        self._mm(self.glob.time_in1, GGML_Q4_K, d, d, self.vec0, self.vec)
        glue.activation(self.vec, self.vec, capi.ACT_SILU, g=g)
        # 5: modulation vectors of every block from silu(vec) (flux_dit.c3:1131-1140),
        # each group of same-shape projections as one launch (at most 64 jobs)
        vec = _t(self.vec)
        dbl = []
        for i, w in enumerate(self.doubles):
            mi = 12 * i
            dbl.append(MatmulJob(_qt(w.img_mod, GGML_Q4_K, 6 * d, d), vec, self.mods[:, mi * d:(mi + 6) * d], 1))
            dbl.append(MatmulJob(_qt(w.txt_mod, GGML_Q4_K, 6 * d, d), vec, self.mods[:, (mi + 6) * d:(mi + 12) * d], 1))
        mi = 12 * len(self.doubles)
        sgl = []
        for w in self.singles:
            sgl.append(MatmulJob(_qt(w.mod, GGML_Q4_K, 3 * d, d), vec, self.mods[:, mi * d:(mi + 3) * d], 1))
            mi += 3
        for jobs, n in ((dbl, 6 * d), (sgl, 3 * d)):
            for k in range(0, len(jobs), 64):
                dispatch_batch_matmul_multi(g, jobs[k:k + 64], n, d)
        self._mm(self.glob.final_mod, GGML_Q4_K, 2 * d, d, self.vec, self.mods[:, mi * d:(mi + 2) * d])
        # 6-8: blocks (flux_dit.c3:1146-1162)
        if self.ahead is not None:
            self.ahead.start(g)
        mi = 0
        try:
            for w in self.doubles:
                self._double(w, self._mod(mi, 6), self._mod(mi + 6, 6))
                mi += 12
            for w in self.singles:
                self._single(w, self._mod(mi, 3))
                mi += 3
        finally:
            # a failed forward leaves no chain half-taken for a later call
            if self.ahead is not None:
                self.ahead.active = False
        # 9: final LayerNorm + adaLN (shift, scale) on the image rows, projection, unpatchify
        fm = self._mod(mi, 2)
        glue.batch_layernorm(hid_i, self.xa[nt:], self.LN_EPS, mod_scale=fm[1], mod_shift=fm[0], g=g)
        self._mm(self.glob.final_linear, GGML_Q4_K, c.patch_dim, d, self.xa[nt:], self.velocity)
        glue.unpatchify(self.velocity, self.out, c.patch, g=g)
        return self.out

    def _multi(self, jobs, N: int, K: int, epilogue: int = capi.EPI_STORE, split: int = 0,
               heads: QkvHeads | None = None) -> None:
        """The blocks' next GEMM group (dispatch_batch_matmul_multi), taking its
        weight images from the chain (and building the following group's)
        when self.ahead is set."""
        if self.ahead is None or not self.ahead.active:  # a block run outside forward(): no chain
            dispatch_batch_matmul_multi(self.g, jobs, N, K, epilogue, split, heads=heads)
            return
        images, nxt = self.ahead.take(jobs, N, K)
        dispatch_batch_matmul_multi(self.g, jobs, N, K, epilogue, split, images=images, next_images=nxt,
                                    heads=heads)

    def _layernorm2(self, scale_t, shift_t, scale_i, shift_i) -> None:
        """LayerNorm + modulation of the joint hidden rows into xa: the text
        rows with the text stream's vectors, the image rows with the image
        stream's, in one launch (two where n_txt % 4 != 0)."""
        nt, g = self.cfg.n_txt, self.g
        if nt % 4 == 0:
            glue.batch_layernorm_split(self.hidden, self.xa, self.LN_EPS, nt, (scale_t, shift_t), (scale_i, shift_i),
                                       g=g)
            return
        for sl, sc, sh in ((slice(0, nt), scale_t, shift_t), (slice(nt, None), scale_i, shift_i)):
            glue.batch_layernorm(self.hidden[sl], self.xa[sl], self.LN_EPS, mod_scale=sc, mod_shift=sh, g=g)

    def _heads(self, norms) -> QkvHeads:
        """The joint Q/K/V as the QKV projections' head routing; norms: per job
        (q_norm, k_norm, first sequence row)."""
        return QkvHeads(self.q, self.k, self.v, self.cfg.n_heads, norms, self.HN_EPS, self.rope)

    def _attention(self, S: int, out: torch.Tensor) -> None:
        """Attention over the joint Q/K/V, its rows written into `out` (the next
        projection's input columns) in out's type."""
        dispatch_flash_attention_rows(self.g, _t(self.q), _t(self.k), _t(self.v), out,
                                      FlashAttentionPC(HEAD_DIM, self.cfg.n_heads, S, 1.0 / math.sqrt(HEAD_DIM)))

    def _double(self, w: FluxDoubleWeights, mi: torch.Tensor, mt: torch.Tensor) -> None:
        """flux_dual_stream_block (flux_dit.c3:746-971). mi / mt: [6, dim]
        (shift1, scale1, gate1, shift2, scale2, gate2) of the image / text
        stream. Each projection multiplies both streams in one launch
        (text rows first, each with its own weight)."""
        c, g = self.cfg, self.g
        d, m, nt, S = c.dim, c.mlp, c.n_txt, c.seq
        ts, im = slice(0, nt), slice(nt, S)
        ni = S - nt

        def jobs(wt, wi, K, x, out, gates=(None, None), out2=None):
            """[text job, image job]: rows ts / im of x, out (and out2)."""
            rows = wt.numel() // (K // 256 * 144)
            return [MatmulJob(_qt(wt, GGML_Q4_K, rows, K), _t(x[ts]), None if out is None else out[ts], nt, 0,
                              gates[0], None if out2 is None else out2[ts]),
                    MatmulJob(_qt(wi, GGML_Q4_K, rows, K), _t(x[im]), None if out is None else out[im], ni, 0,
                              gates[1], None if out2 is None else out2[im])]

        # LayerNorm + modulation of each stream                      (flux_dit.c3:761-779)
        self._layernorm2(mt[1], mt[0], mi[1], mi[0])
        # Q | K | V of both streams, head norm + RoPE into the joint Q/K/V (text
        # rows first) on the projections' result                 (flux_dit.c3:786-863)
        self._multi(jobs(w.txt_qkv, w.img_qkv, d, self.xa, None), 3 * d, d,
                    heads=self._heads([(w.txt_q_norm, w.txt_k_norm, 0), (w.img_q_norm, w.img_k_norm, nt)]))
        # attention rows straight into the projection input             (flux_dit.c3:865-872)
        self._attention(S, self.xa)
        # output projections, hidden += gate1 * proj                  (flux_dit.c3:875-898)
        self._multi(jobs(w.txt_proj, w.img_proj, d, self.xa, self.hidden, (mt[2], mi[2])), d, d,
                    capi.EPI_GATED_RESIDUAL)
        # MLP: LayerNorm + modulation, up + gelu (swiglu: gate and up, silu(gate) * up), down,
        # hidden += gate2 * down (flux_dit.c3:902-967)
        self._layernorm2(mt[4], mt[3], mi[4], mi[3])
        if c.mlp_act == "swiglu":
            self._multi(jobs(w.txt_mlp0, w.img_mlp0, d, self.xa, self.o, out2=self.fa), 2 * m, d,
                        capi.EPI_SPLIT_SWIGLU, split=0)
        else:
            self._multi(jobs(w.txt_mlp0, w.img_mlp0, d, self.xa, self.o, out2=self.fa), m, d,
                        capi.EPI_SPLIT_GELU, split=0)
        self._multi(jobs(w.txt_mlp2, w.img_mlp2, m, self.fa, self.hidden, (mt[5], mi[5])), d, m,
                    capi.EPI_GATED_RESIDUAL)

    def _single(self, w: FluxSingleWeights, mod: torch.Tensor) -> None:
        """flux_single_stream_block (flux_dit.c3:975-1071). mod: [3, dim] (shift, scale, gate)."""
        c, g = self.cfg, self.g
        d, m, S = c.dim, c.mlp, c.seq
        glue.batch_layernorm(self.hidden, self.xa, self.LN_EPS, mod_scale=mod[1], mod_shift=mod[0], g=g)
        # linear1: Q | K | V head-normed and rotated into the joint Q/K/V, and
        # the activated MLP half (gelu; swiglu: silu(gate) * up) straight into
        # linear2's input                                             (flux_dit.c3:1005-1058)
        n1 = 3 * d + c.mlp_in
        self._multi([MatmulJob(_qt(w.linear1, GGML_Q4_K, n1, d), _t(self.xa), None, S, 0, None, self.cat[:, d:])],
                    n1, d, capi.EPI_SPLIT_SWIGLU if c.mlp_act == "swiglu" else capi.EPI_SPLIT_GELU, split=3 * d,
                    heads=self._heads([(w.q_norm, w.k_norm, 0)]))
        self._attention(S, self.cat[:, :d])  # rows into linear2's input  (flux_dit.c3:1042-1047)
        # linear2, hidden += gate * linear2                           (flux_dit.c3:1060-1068)
        self._multi([MatmulJob(_qt(w.linear2, GGML_Q4_K, d, d + m), _t(self.cat), self.hidden, S, 0, mod[2])],
                    d, d + m, capi.EPI_GATED_RESIDUAL)
