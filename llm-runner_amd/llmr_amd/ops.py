"""Host-side mirror of the reference's op interface for the DiT hot path.

The reference's DiT blocks call
    zimage::dispatch_batch_matmul(g, dk, weight, input, output,
                                  out_dim, in_dim, seq_len, row_offset, lora...)
        (dependencies/zimage.c3l/dit.c3:1198-1301, via flux::flux_matmul,
         dependencies/flux.c3l/flux_dit.c3:533-551)
and
    g.dispatch(&dk.flash_attention, {Q, K, V, O}, &FlashAttentionPC, ceil(S/16), H)
        (dependencies/zimage.c3l/dit.c3:1476-1483, flux_dit.c3:1042-1047)
on a RenderGraph (lib/vulkan/graph.c3) over Tensors (lib/model/tensor.c3:8-14).
This module keeps those names and argument meanings; device memory is held in
torch tensors and every op goes through the C-ABI of libllmr_hip.so on the
graph's stream (the caller's current torch stream).
"""
from __future__ import annotations

import ctypes
import dataclasses
import math

import torch

from . import capi
from .gguf import GGML_BF16, GGML_F16, GGML_F32, GGML_Q4_K, GGML_Q8_0, row_bytes

# Largest LoRA rank the backend takes (the reference sizes its scratch for 256:
# DIT_MAX_LORA_RANK, dit.c3:42).
MAX_LORA_RANK = 256

_TORCH_GGML = {torch.float32: GGML_F32, torch.float16: GGML_F16, torch.bfloat16: GGML_BF16}


@dataclasses.dataclass
class Tensor:
    """Device buffer + GGML dtype + logical shape (llm::Tensor, tensor.c3:8-14).

    For quantized types `data` is a uint8 tensor of raw GGUF blocks and
    `shape` is the logical [rows, cols] element shape."""
    data: torch.Tensor
    dtype: int
    shape: tuple

    @staticmethod
    def from_torch(t: torch.Tensor) -> "Tensor":
        return Tensor(t, _TORCH_GGML[t.dtype], tuple(t.shape))

    @staticmethod
    def quantized(blocks: torch.Tensor, ggml_type: int, rows: int, cols: int) -> "Tensor":
        if blocks.dtype != torch.uint8 or blocks.numel() != rows * row_bytes(ggml_type, cols):
            raise ValueError("quantized tensor bytes do not match [rows, cols]")
        return Tensor(blocks, ggml_type, (rows, cols))

    def ptr(self) -> int:
        return self.data.data_ptr()


@dataclasses.dataclass
class FlashAttentionPC:
    """FlashAttentionPC (dependencies/zimage.c3l/dit.c3:136-142)."""
    head_dim: int
    n_heads: int
    seq_len: int
    scale: float


class RenderGraph:
    """The ordering/sync surface of lib/vulkan/graph.c3 for the replaced ops:
    dispatches run in issue order on one stream; checkpoint()/flush() wait
    for them (graph.c3:94-107)."""

    def __init__(self, ctx: capi.Context | None = None, device: int = 0):
        self.ctx = ctx if ctx is not None else capi.Context(device)

    def bind_stream(self) -> None:
        self.ctx.set_stream(torch.cuda.current_stream().cuda_stream)

    def checkpoint(self) -> None:
        self.bind_stream()
        self.ctx.sync()

    flush = checkpoint


def _dev(t: Tensor, what: str) -> None:
    if not t.data.is_cuda:
        raise ValueError(f"{what} must be a device tensor")
    if not t.data.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


@dataclasses.dataclass
class LoraTensor:
    """One linear's LoRA adapter (LoraTensor, lib/model/lora.c3:22-28): a [rank,
    in_dim] and b [out_rows, rank] f32 device tensors; the correction is
    scale * (b . a). `present` goes False once merged into the base weight."""
    a: torch.Tensor
    b: torch.Tensor
    rank: int
    scale: float
    present: bool = True

    def c_struct(self) -> capi.Lora:
        for t, n in ((self.a, "lora.a"), (self.b, "lora.b")):
            if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError(f"{n} must be a contiguous f32 device tensor")
        if self.a.shape[0] != self.rank or self.b.shape[-1] != self.rank:
            raise ValueError("lora.a must be [rank, in_dim] and lora.b [rows, rank]")
        return capi.Lora(self.a.data_ptr(), self.b.data_ptr(), self.rank, float(self.scale))


def dispatch_lora_correction(g: RenderGraph, lora: LoraTensor | None, lora_scratch: torch.Tensor | None,
                             input: Tensor, output: Tensor, in_dim: int, out_dim: int, seq_len: int,
                             b_rows: int = 0, row_offset: int = 0, weight_row_offset: int = 0) -> None:
    """The two-hop LoRA correction on a base output (dispatch_lora_correction,
    dit.c3:1319-1364): output[s, row_offset + o] += scale * (b . (a . input[s]))[
    weight_row_offset + o] for o < b_rows (0: out_dim). No-op without a present
    adapter or with rank > 256, as in the reference. lora_scratch: >= seq_len *
    rank f32 on the device."""
    if lora is None or not lora.present or lora.rank == 0 or lora.rank > MAX_LORA_RANK:
        return
    if lora_scratch is None or lora_scratch.dtype != torch.float32 or not lora_scratch.is_cuda:
        raise ValueError("lora_scratch must be an f32 device tensor")
    if lora_scratch.numel() < seq_len * lora.rank:
        raise ValueError("lora_scratch smaller than seq_len * rank")
    if lora.a.shape[1] != in_dim:
        raise ValueError("lora.a must be [rank, in_dim]")
    rows = b_rows or out_dim
    if weight_row_offset + rows > lora.b.shape[0]:
        raise ValueError("lora.b has fewer rows than weight_row_offset + b_rows")
    for t, n in ((input, "input"), (output, "output")):
        _dev(t, n)
    if output.dtype != GGML_F32:
        raise ValueError("output must be f32")
    if input.data.numel() < seq_len * in_dim or output.data.numel() < seq_len * out_dim:
        raise ValueError("input/output smaller than [seq_len, in_dim] / [seq_len, out_dim]")
    g.bind_stream()
    g.ctx.lora_correction(lora.c_struct(), lora_scratch.data_ptr(), input.ptr(), input.dtype, output.ptr(),
                          in_dim, out_dim, seq_len, b_rows, row_offset, weight_row_offset)


def dispatch_batch_matmul(g: RenderGraph, weight: Tensor, input: Tensor, output: Tensor,
                          out_dim: int, in_dim: int, seq_len: int, row_offset: int,
                          lora: LoraTensor | None = None, lora_scratch: torch.Tensor | None = None,
                          lora_b_rows: int = 0, lora_row_offset: int = 0, lora_weight_row_offset: int = 0) -> None:
    """output[m, n] = sum_k input[m, k] * weight[row_offset + n, k] (f32, overwritten),
    then the LoRA correction when an adapter is present.

    Mirrors zimage::dispatch_batch_matmul (dit.c3:1198-1301) for Q8_0 / Q4_K
    weights, including its trailing dispatch_lora_correction: a GEMM on the
    two-pass kernel (>= 2048 tokens, enough tiles) merges a rank <= 64
    adapter into its 16-bit weight image (W + scale * b a on the adapter's
    output features, rounded once more to 16 bits); otherwise the exact
    correction follows the GEMM."""
    if weight.dtype not in (GGML_Q8_0, GGML_Q4_K):
        raise capi.LlmrError(capi.LLMR_ERR_UNSUPPORTED, f"weight type {weight.dtype}")
    for t, n in ((weight, "weight"), (input, "input"), (output, "output")):
        _dev(t, n)
    if output.dtype != GGML_F32:
        raise ValueError("output must be f32")
    if weight.shape[1] != in_dim or row_offset + out_dim > weight.shape[0]:
        raise ValueError("weight shape does not cover [row_offset, row_offset+out_dim) x in_dim")
    if input.data.numel() < seq_len * in_dim or output.data.numel() < seq_len * out_dim:
        raise ValueError("input/output smaller than [seq_len, in_dim] / [seq_len, out_dim]")
    if lora is not None and lora.present and 0 < lora.rank <= MAX_LORA_RANK:
        # llmr_batch_matmul_lora: on the two-pass GEMM the adapter is merged
        # into the weight image; otherwise the GEMM, then the exact correction
        if lora_scratch is None or lora_scratch.dtype != torch.float32 or not lora_scratch.is_cuda:
            raise ValueError("lora_scratch must be an f32 device tensor")
        if lora_scratch.numel() < seq_len * lora.rank:
            raise ValueError("lora_scratch smaller than seq_len * rank")
        rows = lora_b_rows or out_dim
        if lora.a.shape[1] != in_dim or lora_weight_row_offset + rows > lora.b.shape[0]:
            raise ValueError("lora.a must be [rank, in_dim] and lora.b cover weight_row_offset + b_rows rows")
        g.bind_stream()
        g.ctx.batch_matmul_lora(weight.ptr(), weight.dtype, input.ptr(), input.dtype, output.ptr(), out_dim, in_dim,
                                seq_len, row_offset, lora.c_struct(), lora_scratch.data_ptr(), lora_b_rows,
                                lora_row_offset, lora_weight_row_offset)
        return
    g.bind_stream()
    g.ctx.batch_matmul(weight.ptr(), weight.dtype, input.ptr(), input.dtype, output.ptr(),
                       out_dim, in_dim, seq_len, row_offset)


def merge_one_site(g: RenderGraph, base: Tensor, lora: LoraTensor, dst_row_offset: int = 0) -> bool:
    """Folds a present adapter into a Q8_0 base weight in place (merge_one_site,
    lora_merge.c3:36-73) and marks it merged. Returns False, leaving the adapter
    for the runtime correction, where the reference skips the merge: a non-Q8_0
    base, in_dim % 256 != 0 or rank > 256."""
    if not lora.present:
        return False
    in_dim = base.shape[1]
    if base.dtype != GGML_Q8_0 or in_dim % 256 != 0 or lora.rank > MAX_LORA_RANK:
        return False
    b_rows = lora.b.shape[0]
    if dst_row_offset + b_rows > base.shape[0] or lora.a.shape[1] != in_dim:
        raise ValueError("adapter does not fit the base weight")
    _dev(base, "base")
    lora.c_struct()
    g.bind_stream()
    g.ctx.q8_lora_merge(base.ptr(), lora.a.data_ptr(), lora.b.data_ptr(), in_dim, b_rows, dst_row_offset,
                        lora.rank, lora.scale)
    lora.present = False
    return True


@dataclasses.dataclass
class MatmulJob:
    """One GEMM of dispatch_batch_matmul_multi: input [seq_len, in_dim] times weight
    rows [row_offset, row_offset + out_dim). `output` / `output2` are 2-D device views
    whose row strides become the epilogue's ldy / ldy2 (all jobs of a call must
    share them); `gate` is the GATED_RESIDUAL per-feature gate."""
    weight: Tensor
    input: Tensor
    output: torch.Tensor
    seq_len: int
    row_offset: int = 0
    gate: torch.Tensor | None = None
    output2: torch.Tensor | None = None


def weight_image_bytes(out_dim: int, in_dim: int) -> int:
    """Bytes of the 16-bit weight image of out_dim rows of in_dim (llmr_weight_image_bytes)."""
    n = capi.lib().llmr_weight_image_bytes(out_dim, in_dim)
    if n == 0:
        raise ValueError("weight images need in_dim % 64 == 0")
    return n


def swiglu_weight_image_bytes(n_out: int, in_dim: int) -> int:
    """Bytes of the SwiGLU-arranged image of n_out outputs (their gate and up
    rows) of in_dim (llmr_swiglu_weight_image_bytes)."""
    n = capi.lib().llmr_swiglu_weight_image_bytes(n_out, in_dim)
    if n == 0:
        raise ValueError("weight images need in_dim % 64 == 0")
    return n


def split_swiglu_image_bytes(split: int, f: int, in_dim: int) -> int:
    """Bytes of a SPLIT_SWIGLU job's image: the plain image of its first
    `split` rows, then the SwiGLU image of its f outputs."""
    return (weight_image_bytes(split, in_dim) if split else 0) + swiglu_weight_image_bytes(f, in_dim)


def build_weight_image(g: RenderGraph, weight: Tensor, out_dim: int, in_dim: int, row_offset: int,
                       input_dtype: int, image: torch.Tensor) -> None:
    """Rows [row_offset, row_offset + out_dim) of `weight` dequantized into
    `image` (a device tensor of at least weight_image_bytes bytes) as the
    two-pass GEMM's operands for input_dtype (F16 or BF16), on the current
    stream; pass it to dispatch_batch_matmul_multi(images=...)."""
    _dev(weight, "weight")
    if weight.shape[1] != in_dim or row_offset + out_dim > weight.shape[0]:
        raise ValueError("weight shape does not cover [row_offset, row_offset+out_dim) x in_dim")
    if not image.is_cuda or not image.is_contiguous():
        raise ValueError("image must be a contiguous device tensor")
    g.bind_stream()
    g.ctx.build_weight_image(weight.ptr(), weight.dtype, input_dtype, out_dim, in_dim, row_offset,
                             image.data_ptr(), image.numel() * image.element_size())


@dataclasses.dataclass
class QkvHeads:
    """Head routing of a QKV projection's Q | K | V columns (llmr_qkv_heads_out):
    q, k, v [n_heads, seq, 128] f16 / bf16 device tensors, the RoPE tables
    (cos, sin f32 [seq, 64]) or None, and per job (q_norm, k_norm, row0):
    its head-norm weights ([128] f32 or None) and the sequence position of its
    token 0."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    n_heads: int
    jobs: list
    eps: float = 1e-6
    rope: tuple | None = None


def _qkv_heads_out(h: QkvHeads, n_jobs: int) -> tuple:
    H, S, D = h.q.shape
    if D != 128 or H != h.n_heads or h.k.shape != h.q.shape or h.v.shape != h.q.shape:
        raise ValueError("q/k/v must be [n_heads, seq, 128] alike")
    if not (h.q.dtype == h.k.dtype == h.v.dtype) or h.q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q/k/v must share one dtype, float16 or bfloat16")
    if not all(t.is_contiguous() and t.is_cuda for t in (h.q, h.k, h.v)):
        raise ValueError("q/k/v must be contiguous device tensors")
    if len(h.jobs) != n_jobs:
        raise ValueError("one (q_norm, k_norm, row0) per job")

    def vec(t, what, n):
        if t is None:
            return None
        if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous() or t.numel() < n:
            raise ValueError(f"{what} must be a contiguous f32 device tensor of {n} elements")
        return t.data_ptr()

    cos_p = sin_p = None
    if h.rope is not None:
        cos_p = vec(h.rope[0], "rope_cos", S * 64)
        sin_p = vec(h.rope[1], "rope_sin", S * 64)
    hj = [capi.QkvHeadsJob(vec(qn, "q_norm", 128), vec(kn, "k_norm", 128), row0) for qn, kn, row0 in h.jobs]
    out = capi.QkvHeadsOut(h.q.data_ptr(), h.k.data_ptr(), h.v.data_ptr(), _TORCH_GGML[h.q.dtype], H, S,
                           float(h.eps), cos_p, sin_p, None)
    return out, hj


@dataclasses.dataclass
class NextImage:
    """One weight image a call builds for a later call: rows [row_offset,
    row_offset + out_dim) of `weight` (a quantized Tensor) with in_dim
    columns, into `image` (a device tensor of weight_image_bytes); swiglu:
    the SwiGLU arrangement of out_dim outputs whose gate rows start at
    row_offset and up rows up_offset rows later (0: out_dim;
    swiglu_weight_image_bytes)."""
    weight: Tensor
    out_dim: int
    in_dim: int
    image: object
    row_offset: int = 0
    swiglu: bool = False
    up_offset: int = 0

    def nbytes(self) -> int:
        return (swiglu_weight_image_bytes if self.swiglu else weight_image_bytes)(self.out_dim, self.in_dim)

    def rows(self) -> int:
        if not self.swiglu:
            return self.row_offset + self.out_dim
        return self.row_offset + (self.up_offset or self.out_dim) + self.out_dim


@dataclasses.dataclass
class NextImages:
    """Weight images of the GEMM groups issued next (llmr_next_weight_images):
    1 to 8 NextImage entries, weights of one type."""
    entries: list

    @classmethod
    def group(cls, weights, out_dim: int, in_dim: int, images, row_offsets=(0, 0)) -> "NextImages":
        """One group's images: its weights, out_dim x in_dim each."""
        return cls([NextImage(w, out_dim, in_dim, im, ro) for w, im, ro in zip(weights, images, row_offsets)])

    @classmethod
    def split_swiglu(cls, weights, split: int, f: int, in_dim: int, images, row_offsets=(0, 0)) -> "NextImages":
        """A SPLIT_SWIGLU group's images (out_dim = split + 2 f): per weight,
        the plain image of its first split rows (none when split is 0) and,
        in the same buffer right after it, the SwiGLU image of its f outputs."""
        es = []
        for w, im, ro in zip(weights, images, row_offsets):
            flat = im.view(torch.uint8).reshape(-1)
            plain = weight_image_bytes(split, in_dim) if split else 0
            if split:
                es.append(NextImage(w, split, in_dim, flat[:plain], ro))
            es.append(NextImage(w, f, in_dim, flat[plain:], ro + split, True))
        return cls(es)

    def __add__(self, other: "NextImages") -> "NextImages":
        return NextImages(self.entries + other.entries)


def _next_images_struct(next_images: NextImages) -> capi.NextWeightImages:
    es = next_images.entries
    if not 1 <= len(es) <= 8:
        raise ValueError("next_images: one to eight images")
    if len(es) != len(set(e.image.data_ptr() for e in es)):
        raise ValueError("next_images: one buffer per image")
    nt = es[0].weight.dtype
    arr = (capi.NextWeightImage * 8)()
    for i, e in enumerate(es):
        _dev(e.weight, "next weight")
        nbytes = e.nbytes()
        if e.weight.dtype != nt or e.weight.shape[1] != e.in_dim or e.rows() > e.weight.shape[0]:
            raise ValueError("next weights: one type, covering the image's rows x in_dim")
        if not e.image.is_cuda or e.image.numel() * e.image.element_size() < nbytes:
            raise ValueError(f"next images must be device tensors of at least {nbytes} bytes")
        arr[i] = capi.NextWeightImage(e.weight.ptr(), e.out_dim, e.in_dim, e.row_offset, int(e.swiglu), e.up_offset,
                                      e.image.data_ptr(), e.image.numel() * e.image.element_size())
    return capi.NextWeightImages(nt, len(es), arr)


def build_next_images(g: RenderGraph, next_images: NextImages, input_dtype: int) -> None:
    """The images of next_images built now, on the current stream, for
    input_dtype (F16 or BF16): a llmr_batch_matmul_multi_images call with no
    jobs (plain and SwiGLU-arranged images alike)."""
    nx = _next_images_struct(next_images)
    g.bind_stream()
    g.ctx.batch_matmul_multi_images(next_images.entries[0].weight.dtype, input_dtype, 0, 0, [], None, None, nx)


def dispatch_batch_matmul_multi(g: RenderGraph, jobs: list, out_dim: int, in_dim: int,
                                epilogue: int = capi.EPI_STORE, split: int = 0, images=None,
                                next_images: NextImages | None = None, heads: QkvHeads | None = None) -> None:
    """The jobs' GEMMs with a shared epilogue (llmr_batch_matmul_multi): a plain
    store, `output += gate * result` (gated_residual_linear), a column split
    whose features >= split are GELU'd into output2 (linear1's MLP half feeding
    linear2, flux_dit.c3:1049-1058), or a column split whose last 2 f
    features are a SwiGLU gate and up, silu(gate) * up into output2's f
    columns (the Flux.2 linear1 and MLP in-projection, flux_dit.c3:917-931,
    1013-1018; output may be None when split is 0). Pairs of jobs run as one launch; a
    group of Q4_K jobs of at most 4 tokens with a plain store (the per-block
    modulation projections) runs as one GEMV launch. images: None, or one
    device tensor per job holding the job's weight image (build_weight_image
    or an earlier call's next_images, same weight, row_offset and input
    type), used where a pair runs two-pass; next_images: images of later
    groups (NextImages), built partly by this call's idle workgroups and
    complete when the stream's next call starts
    (llmr_batch_matmul_multi_images). heads: the
    Q | K | V columns (all of a plain store, [0, split) of a split) head-normed,
    rotated and written head-major into heads.q/k/v instead of `output`, which
    may then be None (llmr_batch_matmul_multi_qkv; batch_head_norm +
    transpose_heads + mrope after the QKV projection, flux_dit.c3:786-863)."""
    if not jobs:
        return
    wtype, xtype = jobs[0].weight.dtype, jobs[0].input.dtype

    def stride(t):
        # a one-row view writes row 0 only, so it fits any common row stride
        if t.dim() != 2 or t.stride(1) != 1:
            raise ValueError("outputs must be 2-D views with contiguous rows")
        return t.stride(0) if t.shape[0] > 1 else None

    def common_stride(views, what):
        strides = {stride(t) for t in views} - {None}
        if len(strides) > 1:
            raise ValueError(f"{what} views must share one row stride")
        return strides.pop() if strides else (views[0].shape[1] + 3) // 4 * 4

    swiglu = epilogue == capi.EPI_SPLIT_SWIGLU
    no_out = (swiglu and split == 0) or heads is not None
    if no_out:
        ldy = 0
    else:
        ldy = common_stride([j.output for j in jobs], "output")
    has2 = [j.output2 is not None for j in jobs]
    if any(has2) and not all(has2):
        raise ValueError("either every job has output2 or none")
    ldy2 = common_stride([j.output2 for j in jobs], "output2") if has2[0] else 0
    o2type = _TORCH_GGML.get(jobs[0].output2.dtype, 0) if has2[0] else 0
    cj = []
    for j in jobs:
        if j.weight.dtype != wtype or j.input.dtype != xtype:
            raise ValueError("all jobs share the weight and input types")
        _dev(j.weight, "weight")
        _dev(j.input, "input")
        if j.weight.shape[1] != in_dim or j.row_offset + out_dim > j.weight.shape[0]:
            raise ValueError("weight shape does not cover [row_offset, row_offset+out_dim) x in_dim")
        if j.input.data.numel() < j.seq_len * in_dim:
            raise ValueError("input smaller than [seq_len, in_dim]")
        if not no_out:
            if not j.output.is_cuda or j.output.dtype != torch.float32:
                raise ValueError("outputs must be f32 device views")
            width = split if epilogue in (capi.EPI_SPLIT_GELU, capi.EPI_SPLIT_SWIGLU) else out_dim
            if j.output.shape[0] < j.seq_len or j.output.shape[1] < width:
                raise ValueError("output view smaller than [seq_len, out_dim]")
        o2 = 0
        if j.output2 is not None:
            if _TORCH_GGML.get(j.output2.dtype) != o2type:
                raise ValueError("output2 views must share one dtype")
            width2 = (out_dim - split) // 2 if swiglu else out_dim - split
            if j.output2.shape[0] < j.seq_len or j.output2.shape[1] < width2:
                raise ValueError(f"output2 view smaller than [seq_len, {width2}]")
            o2 = j.output2.data_ptr()
        gp = 0
        if j.gate is not None:
            if j.gate.dtype != torch.float32 or not j.gate.is_contiguous() or j.gate.numel() < out_dim:
                raise ValueError("gate must be a contiguous f32 vector of out_dim elements")
            gp = j.gate.data_ptr()
        cj.append(capi.MatmulJob(j.weight.ptr(), j.input.ptr(), None if no_out else j.output.data_ptr(),
                                 gp or None, o2 or None, j.seq_len, j.row_offset))
    epi = capi.MatmulEpilogue(epilogue, ldy, split, ldy2, o2type)
    hout = _qkv_heads_out(heads, len(jobs)) if heads is not None else None
    g.bind_stream()
    if images is None and next_images is None and hout is None:
        g.ctx.batch_matmul_multi(wtype, xtype, out_dim, in_dim, cj, epi)
        return
    ptrs = None
    if images is not None:
        if len(images) != len(jobs):
            raise ValueError("one weight image per job")
        if epilogue == capi.EPI_SPLIT_SWIGLU:
            need = split_swiglu_image_bytes(split, (out_dim - split) // 2, in_dim)
        else:
            need = weight_image_bytes(out_dim, in_dim)
        for im in images:
            if not im.is_cuda or im.numel() * im.element_size() < need:
                raise ValueError(f"weight images must be device tensors of at least {need} bytes")
        ptrs = [im.data_ptr() for im in images]
    nx = _next_images_struct(next_images) if next_images is not None else None
    if hout is not None:
        g.ctx.batch_matmul_multi_qkv(wtype, xtype, out_dim, in_dim, cj, epi, hout[0], hout[1], ptrs, nx)
    else:
        g.ctx.batch_matmul_multi_images(wtype, xtype, out_dim, in_dim, cj, epi, ptrs, nx)


def dispatch_batch_matmul_swiglu(g: RenderGraph, weight_gate: Tensor, weight_up: Tensor,
                                 input: Tensor, output: Tensor, out_dim: int, in_dim: int,
                                 seq_len: int) -> None:
    """output[s, o] = silu(input . weight_gate[o]) * (input . weight_up[o]) (f32, overwritten).

    Mirrors the batch_matmul_swiglu_q8 dispatch of dit_transformer_layer
    (dit.c3:1562-1580): both weights Q8_0 [out_dim, in_dim], rows from 0. The
    reference takes this path only without LoRA on gate/up; a present LoRA
    keeps the caller's two-matmul fallback (dit.c3:1582-1592)."""
    if weight_gate.dtype != GGML_Q8_0 or weight_up.dtype != GGML_Q8_0:
        raise capi.LlmrError(capi.LLMR_ERR_UNSUPPORTED, "SwiGLU GEMM needs Q8_0 gate and up weights")
    for t, n in ((weight_gate, "weight_gate"), (weight_up, "weight_up"), (input, "input"),
                 (output, "output")):
        _dev(t, n)
    if output.dtype != GGML_F32:
        raise ValueError("output must be f32")
    for w in (weight_gate, weight_up):
        if w.shape[1] != in_dim or out_dim > w.shape[0]:
            raise ValueError("weight shape does not cover out_dim x in_dim")
    if input.data.numel() < seq_len * in_dim or output.data.numel() < seq_len * out_dim:
        raise ValueError("input/output smaller than [seq_len, in_dim] / [seq_len, out_dim]")
    g.bind_stream()
    g.ctx.batch_matmul_swiglu(weight_gate.ptr(), weight_up.ptr(), weight_gate.dtype, input.ptr(),
                              input.dtype, output.ptr(), out_dim, in_dim, seq_len)


def dispatch_flash_attention(g: RenderGraph, q: Tensor, k: Tensor, v: Tensor, out: Tensor,
                             pc: FlashAttentionPC) -> None:
    """out[s, h*D + d] = softmax(scale * q k^T) v per head; q/k/v [H, S, D], out f32 [S, H*D]."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out")):
        _dev(t, n)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    if out.dtype != GGML_F32:
        raise ValueError("out must be f32")
    n = pc.n_heads * pc.seq_len * pc.head_dim
    if min(q.data.numel(), k.data.numel(), v.data.numel(), out.data.numel()) < n:
        raise ValueError("buffers smaller than [n_heads, seq_len, head_dim]")
    g.bind_stream()
    g.ctx.flash_attention(q.ptr(), k.ptr(), v.ptr(), q.dtype, out.ptr(), pc.head_dim, pc.n_heads,
                          pc.seq_len, pc.scale)


def dispatch_flash_attention_rows(g: RenderGraph, q: Tensor, k: Tensor, v: Tensor, out: torch.Tensor,
                                  pc: FlashAttentionPC) -> None:
    """dispatch_flash_attention with the output rows written into `out`, a 2-D
    device view [seq_len, >= n_heads * head_dim] of f32, f16 or bf16 with
    contiguous rows (e.g. the columns of the next projection's input),
    rounded to nearest even (llmr_flash_attention_rows)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dev(t, n)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    ot = _TORCH_GGML.get(out.dtype)
    if ot is None or not out.is_cuda or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError("out must be a 2-D f32/f16/bf16 device view with contiguous rows")
    if out.shape[0] < pc.seq_len or out.shape[1] < pc.n_heads * pc.head_dim:
        raise ValueError("out view smaller than [seq_len, n_heads * head_dim]")
    n = pc.n_heads * pc.seq_len * pc.head_dim
    if min(q.data.numel(), k.data.numel(), v.data.numel()) < n:
        raise ValueError("buffers smaller than [n_heads, seq_len, head_dim]")
    g.bind_stream()
    g.ctx.flash_attention_rows(q.ptr(), k.ptr(), v.ptr(), q.dtype, out.data_ptr(), ot, out.stride(0), pc.head_dim,
                               pc.n_heads, pc.seq_len, pc.scale)


# ---- torch-tensor conveniences (tests, bench) --------------------------------

_default_graph: RenderGraph | None = None


def default_graph() -> RenderGraph:
    global _default_graph
    if _default_graph is None:
        _default_graph = RenderGraph()
    return _default_graph


def batch_matmul(w_blocks: torch.Tensor, wtype: int, x: torch.Tensor, out_dim: int,
                 row_offset: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [M, K] (f32/f16/bf16, cuda) times rows [row_offset, row_offset+out_dim) of the
    quantized weight -> f32 [M, out_dim]."""
    M, K = x.shape
    rows = w_blocks.numel() // row_bytes(wtype, K)
    if out is None:
        out = torch.empty((M, out_dim), dtype=torch.float32, device=x.device)
    dispatch_batch_matmul(default_graph(), Tensor.quantized(w_blocks, wtype, rows, K),
                          Tensor.from_torch(x), Tensor.from_torch(out), out_dim, K, M, row_offset)
    return out


def batch_matmul_swiglu(wg_blocks: torch.Tensor, wu_blocks: torch.Tensor, x: torch.Tensor,
                        out_dim: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [M, K] (f32/f16/bf16, cuda) and Q8_0 gate/up weights [out_dim, K] ->
    f32 [M, out_dim] = silu(x Wg^T) * (x Wu^T)."""
    M, K = x.shape
    if out is None:
        out = torch.empty((M, out_dim), dtype=torch.float32, device=x.device)
    rows_g = wg_blocks.numel() // row_bytes(GGML_Q8_0, K)
    rows_u = wu_blocks.numel() // row_bytes(GGML_Q8_0, K)
    dispatch_batch_matmul_swiglu(default_graph(), Tensor.quantized(wg_blocks, GGML_Q8_0, rows_g, K),
                                 Tensor.quantized(wu_blocks, GGML_Q8_0, rows_u, K),
                                 Tensor.from_torch(x), Tensor.from_torch(out), out_dim, K, M)
    return out


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """q, k, v [H, S, 128] -> f32 [S, H*128]."""
    H, S, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty((S, H * D), dtype=torch.float32, device=q.device)
    dispatch_flash_attention(default_graph(), Tensor.from_torch(q), Tensor.from_torch(k),
                             Tensor.from_torch(v), Tensor.from_torch(out),
                             FlashAttentionPC(D, H, S, scale))
    return out


def dequant(w_blocks: torch.Tensor, wtype: int, n_rows: int, in_dim: int,
            row_offset: int = 0) -> torch.Tensor:
    out = torch.empty((n_rows, in_dim), dtype=torch.float32, device=w_blocks.device)
    g = default_graph()
    g.bind_stream()
    g.ctx.dequant(w_blocks.data_ptr(), wtype, n_rows, in_dim, row_offset, out.data_ptr())
    return out


def dequant_operand_f16(w_blocks: torch.Tensor, wtype: int, n_rows: int, in_dim: int,
                        row_offset: int = 0) -> torch.Tensor:
    out = torch.empty((n_rows, in_dim), dtype=torch.int16, device=w_blocks.device)
    g = default_graph()
    g.bind_stream()
    g.ctx.dequant_operand_f16(w_blocks.data_ptr(), wtype, n_rows, in_dim, row_offset,
                              out.data_ptr())
    return out
