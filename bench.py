"""Benchmark of the DiT hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                    [--components a,b,...] [--no-cpu-baseline]
    python bench.py --library-baselines [--steps K] [--warmup W]

A step is one pass of the hot path over one batch of synthetic input already
resident in HBM: for the default workload `flux_attention` one non-causal
attention call at the Flux shape (H=24, S=4608, D=128, f16, RoPE applied),
for a GEMM workload one dequant-GEMM call, each through the C-ABI with device
pointers (what a compiled caller issues per step). Rank 0 prints one JSON line:
`value` is the workload's TFLOP/s (4*H*S^2*D or 2*M*N*K per step), timed
with HIP events on the stream the kernels run on; `components` carries the
same measurement for the other configurations (Q4_K Flux linears, the Q8_0
linear, the Z-Image QKV and SwiGLU projections) and the composed ones: one
full Z-Image block and one Flux-dev-shaped denoising step (ms/step), so the
three-part headline metric is reported in one line. `roofline` describes the workload's kernel,
`cpu_baseline` the oracle timed on a bounded sample on the host cores.
Every measurement runs its step back to back for DEVICE_WARMUP_MS of GPU
time before the W warmup and K timed steps (the GPU's clock settles only
after some tens of milliseconds of load); `cold_ms_per_step` is the
headline's K steps timed straight after set-up and W warmup steps, without
that.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "llm-runner_amd"))

METRIC = "Q4_K/Q8_0 dequant-GEMM TFLOPS, flash-attn TFLOPS, Flux 1024² ms/step"
# MI355X dense fp16/bf16 MFMA: 256 CUs x 2.4 GHz x 4096 flop per clock
# (the 2.5 PFLOP/s published figure, unrounded)
PEAK_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, published
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")


# Sustained load first runs the GPU below its steady clock: on MI355X the
# flash-attention launch takes ~306 us over its first 20 steps, ~287 over the
# next 20 and settles at ~261 after ~100 (~30 ms), with the shader clock read
# between steps dipping to ~2.0 GHz and returning to ~2.4 GHz. Each
# measurement therefore first runs its step back to back for this much GPU
# time (at most DEVICE_WARMUP_MAX_STEPS steps: after ~11k back-to-back calls
# of the 28 us few-token GEMM, each of three launches, its later steps ran
# 2-4x slower, which 3.7k calls did not do), then the W warmup steps and the
# K timed steps.
DEVICE_WARMUP_MS = 100.0
DEVICE_WARMUP_MAX_STEPS = 2000


def _device_warmup(fn, min_ms: float = DEVICE_WARMUP_MS):
    """Runs `fn` back to back for about `min_ms` of GPU time (untimed, at most
    DEVICE_WARMUP_MAX_STEPS steps); returns the number of steps run."""
    import torch
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    fn()
    b.record(st)
    torch.cuda.synchronize()
    n = min(DEVICE_WARMUP_MAX_STEPS, max(1, math.ceil(min_ms / max(a.elapsed_time(b), 1e-3)))) - 1
    for _ in range(n):
        fn()
    torch.cuda.synchronize()
    return n + 1


def _time_steps(fn, steps: int, warmup: int, per_step: bool = False):
    """Runs warmup + timed steps; returns (total ms over `steps`, per-step ms
    list or None). The total is timed between two events only: an event
    recorded after every step adds a few microseconds of stream time per
    step, a sixth of a 16 us launch. With per_step, `steps` more steps run
    with an event after each, for the per-step list."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(steps):
        fn()
    b.record(st)
    torch.cuda.synchronize()
    per = None
    if per_step:
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        evs[0].record(st)
        for i in range(steps):
            fn()
            evs[i + 1].record(st)
        torch.cuda.synchronize()
        per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    return a.elapsed_time(b), per


def _traffic(name: str):
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def _bound_ctx():
    """The library context bound to the current stream. Kernel-level steps call
    the C-ABI with device pointers resolved once, as a compiled caller (the
    reference's C3 host) does; the Python checks of llmr_amd.ops run once in
    set-up, not per step."""
    from llmr_amd import ops
    g = ops.default_graph()
    g.bind_stream()
    return g.ctx


def setup_attention(dev, f32: bool = False):
    """The Flux attention; with f32, Q/K/V are handed over as f32 (the
    reference's buffer type, rounded to fp16 by the backend)."""
    import torch
    from llmr_amd import ops, workloads
    a = workloads.FLUX_ATTENTION
    q, k, v = workloads.attention_inputs(a)
    qt, kt, vt = (torch.from_numpy(t).to(dev) for t in (q, k, v))
    if f32:
        qt, kt, vt = (t.float() for t in (qt, kt, vt))
    out = torch.empty((a.S, a.H * a.D), dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(a.D)
    ops.flash_attention(qt, kt, vt, scale, out=out)  # the checked host path once
    ctx, xt = _bound_ctx(), ops.Tensor.from_torch(qt).dtype
    ptrs = (qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), xt, out.data_ptr(), a.D, a.H, a.S, scale)

    def step():
        ctx.flash_attention(*ptrs)

    cfg = {"workload": "flux_attention_f32" if f32 else "flux_attention", "heads": a.H, "seq_len": a.S,
           "head_dim": a.D, "qkv_dtype": "f32" if f32 else "f16",
           "rope": "3-axis 16/56/56 theta=1e4, applied beforehand", "causal": False}
    nbytes = a.bytes + (3 * a.H * a.S * a.D * 2 if f32 else 0)  # f32 Q/K/V: twice the input bytes
    return step, a.flops, nbytes, cfg, "f16"


def setup_lora(dev):
    """The two-hop LoRA correction (rank 32, scale 1) on the Flux single-block
    linear1 output: 4608 tokens, 3072 -> 21504, bf16 input, f32 output."""
    import torch
    from llmr_amd import ops
    seq, in_dim, out_dim, rank = 4608, 3072, 21504, 32
    gen = torch.Generator(device="cpu").manual_seed(7)
    a = (0.02 * torch.randn(rank, in_dim, generator=gen)).to(dev)
    b = (0.02 * torch.randn(out_dim, rank, generator=gen)).to(dev)
    lora = ops.LoraTensor(a, b, rank, 1.0)
    x = torch.randn(seq, in_dim, generator=gen).bfloat16().to(dev)
    y = torch.zeros(seq, out_dim, device=dev)
    scratch = torch.empty(seq * rank, device=dev)
    g = ops.default_graph()
    xt, yt = ops.Tensor.from_torch(x), ops.Tensor.from_torch(y)

    def step():
        ops.dispatch_lora_correction(g, lora, scratch, xt, yt, in_dim, out_dim, seq)

    flops = 2.0 * seq * rank * (in_dim + out_dim)
    nbytes = seq * in_dim * 2 + rank * in_dim * 4 + out_dim * rank * 4 + 2 * seq * rank * 4 + 2 * seq * out_dim * 4
    cfg = {"workload": "lora_flux_linear1", "seq_len": seq, "in_dim": in_dim, "out_dim": out_dim, "rank": rank,
           "input": "bf16", "output": "f32 (accumulated)"}
    return step, flops, nbytes, cfg, "f32"


def setup_gemm(dev, name):
    import torch
    from llmr_amd import gguf, ops, workloads
    g = workloads.GEMMS[name]
    blk = workloads.gemm_weight_blocks(g)
    x = workloads.gemm_activations_f32(g)
    w = torch.from_numpy(blk).to(dev)
    xt = torch.from_numpy(x)
    xt = {gguf.GGML_F32: xt, gguf.GGML_F16: xt.half(), gguf.GGML_BF16: xt.bfloat16()}[g.xtype].to(dev)
    out = torch.empty((g.M, g.N), dtype=torch.float32, device=dev)
    ops.batch_matmul(w, g.wtype, xt, g.N, out=out)  # the checked host path once
    ctx = _bound_ctx()
    ptrs = (w.data_ptr(), g.wtype, xt.data_ptr(), ops.Tensor.from_torch(xt).dtype, out.data_ptr(), g.N, g.K, g.M, 0)

    def step():
        ctx.batch_matmul(*ptrs)

    cfg = {"workload": name, "M": g.M, "N": g.N, "K": g.K, "weight": gguf.TYPE_NAMES[g.wtype],
           "activations": gguf.TYPE_NAMES[g.xtype].lower(), "output": "f32"}
    # MFMA operand type: bf16 activations run bf16 MFMA, f32/f16 ones fp16 MFMA
    return step, g.flops, g.bytes, cfg, "bf16" if g.xtype == gguf.GGML_BF16 else "f16"


def setup_gemm_lora(dev):
    """flux_linear1 (Q4_K, 4608 x 21504 x 3072, bf16) with a rank-32 LoRA on
    its whole output through llmr_batch_matmul_lora: the adapter is merged into
    the two-pass GEMM's 16-bit weight image as the image is built. Its time
    against flux_linear1's is the adapter's cost."""
    import torch
    from llmr_amd import capi, gguf, ops, workloads
    g = workloads.GEMMS["flux_linear1"]
    rank = 32
    w = torch.from_numpy(workloads.gemm_weight_blocks(g)).to(dev)
    xt = torch.from_numpy(workloads.gemm_activations_f32(g)).bfloat16().to(dev)
    gen = torch.Generator(device="cpu").manual_seed(7)
    a = (0.02 * torch.randn(rank, g.K, generator=gen)).to(dev)
    b = (0.02 * torch.randn(g.N, rank, generator=gen)).to(dev)
    lora = ops.LoraTensor(a, b, rank, 1.0)
    out = torch.empty((g.M, g.N), dtype=torch.float32, device=dev)
    scratch = torch.empty(g.M * rank, device=dev)
    gr = ops.default_graph()
    wt = ops.Tensor.quantized(w, g.wtype, g.N, g.K)
    ops.dispatch_batch_matmul(gr, wt, ops.Tensor.from_torch(xt), ops.Tensor.from_torch(out), g.N, g.K, g.M, 0,
                              lora=lora, lora_scratch=scratch)  # the checked host path once
    ctx = _bound_ctx()
    lc = lora.c_struct()
    args = (w.data_ptr(), g.wtype, xt.data_ptr(), gguf.GGML_BF16, out.data_ptr(), g.N, g.K, g.M, 0, lc,
            scratch.data_ptr())

    def step():
        ctx.batch_matmul_lora(*args)

    flops = g.flops + 2.0 * g.M * rank * (g.K + g.N)
    cfg = {"workload": "flux_linear1_lora", "M": g.M, "N": g.N, "K": g.K, "weight": "Q4_K", "activations": "bf16",
           "output": "f32", "lora_rank": rank}
    return step, flops, g.bytes, cfg, "bf16"


def setup_swiglu(dev, name):
    import torch
    from llmr_amd import gguf, ops, workloads
    g = workloads.SWIGLUS[name]
    wg = torch.from_numpy(workloads.gemm_weight_blocks(g)).to(dev)
    wu = torch.from_numpy(workloads.swiglu_up_blocks(g)).to(dev)
    xt = torch.from_numpy(workloads.gemm_activations_f32(g))
    xt = {gguf.GGML_F32: xt, gguf.GGML_F16: xt.half(), gguf.GGML_BF16: xt.bfloat16()}[g.xtype].to(dev)
    out = torch.empty((g.M, g.N), dtype=torch.float32, device=dev)
    ops.batch_matmul_swiglu(wg, wu, xt, g.N, out=out)  # the checked host path once
    ctx = _bound_ctx()
    ptrs = (wg.data_ptr(), wu.data_ptr(), g.wtype, xt.data_ptr(), ops.Tensor.from_torch(xt).dtype, out.data_ptr(),
            g.N, g.K, g.M)

    def step():
        ctx.batch_matmul_swiglu(*ptrs)

    cfg = {"workload": name, "M": g.M, "N": g.N, "K": g.K, "weight": "Q8_0 gate + up",
           "activations": gguf.TYPE_NAMES[g.xtype].lower(), "output": "f32 silu(gate) * up"}
    return step, g.flops, g.bytes, cfg, "bf16" if g.xtype == gguf.GGML_BF16 else "f16"


def setup_zimage_block(dev):
    """One Z-Image DiT block at full size (hidden 3840, 30 heads, FFN 10240,
    4096 image + 256 text tokens), Q8_0 weights, bf16 activations."""
    import torch
    from llmr_amd import dit, synth, workloads
    dim, H, ffn = 3840, 30, 10240
    a = workloads.ZIMAGE_ATTENTION
    S = a.S
    w = dit.zimage_layer_weights(dim, H, ffn, device=dev)
    cos_t, sin_t = workloads.rope_tables(workloads.attention_positions(a), a.axes, a.theta)
    rope = (torch.from_numpy(cos_t).to(dev), torch.from_numpy(sin_t).to(dev))
    h0 = workloads.round_bf16(synth.normal(workloads.SEED, 10, S * dim).reshape(S, dim))
    hidden = torch.from_numpy(h0).to(dev)
    blk = dit.ZImageBlock(dim, H, ffn, S, act_dtype=torch.bfloat16, device=dev)

    def step():
        blk.forward(w, hidden, *rope)

    flops = 2.0 * S * dim * (3 * dim + dim + 2 * ffn + ffn) + a.flops
    cfg = {"workload": "zimage_block", "hidden": dim, "heads": H, "head_dim": 128, "ffn": ffn, "seq_len": S,
           "weights": "Q8_0", "activations": "bf16", "sequence": "rmsnorm*scale, qkv, headnorm+rope, attention, "
           "o-proj, postnorm+tanh-gated residual, rmsnorm*scale, swiglu, down, postnorm+tanh-gated residual"}
    return step, flops, None, cfg, "bf16"


def setup_zimage_block_c3(dev):
    """The Z-Image block at the same full size as a compiled C caller with the
    reference's buffer types issues it: the call order of the C11 harness
    tests/c/zimage_layer.c (dit.c3:1421-1610), f32 activation buffers
    throughout, each GEMM through llmr_batch_matmul_pc (the QKV projection
    over the fused weight), the SwiGLU through llmr_batch_matmul_swiglu_pc,
    head norm + RoPE + transpose into f32 Q/K/V by llmr_qkv_heads, attention
    through llmr_flash_attention_pc, norms and gated residuals by the glue
    entry points. Device pointers and push constants are resolved once."""
    import ctypes

    import torch
    from llmr_amd import capi, dit, synth, workloads
    from llmr_amd.gguf import GGML_Q8_0
    dim, H, ffn = 3840, 30, 10240
    a = workloads.ZIMAGE_ATTENTION
    S, eps = a.S, dit.ZImageBlock.EPS
    w = dit.zimage_layer_weights(dim, H, ffn, device=dev)
    cos_t, sin_t = (torch.from_numpy(t).to(dev) for t in
                    workloads.rope_tables(workloads.attention_positions(a), a.axes, a.theta))
    hidden = torch.from_numpy(synth.normal(workloads.SEED, 10, S * dim).reshape(S, dim)).to(dev)
    f32 = dict(dtype=torch.float32, device=dev)
    buf_a, qkv, attn, t = (torch.empty(S, n, **f32) for n in (dim, 3 * dim, dim, dim))
    f = torch.empty(S, ffn, **f32)
    qh, kh, vh = (torch.empty(H, S, 128, **f32) for _ in range(3))
    ctx = _bound_ctx()
    lib, h, F32, Q8 = capi.lib(), ctx.handle, 0, GGML_Q8_0
    p = {k: v.data_ptr() for k, v in vars(w).items() if isinstance(v, torch.Tensor)}
    pc_qkv = capi.BatchMatMulParams(3 * dim, dim, S, 0)
    pc_o = capi.BatchMatMulParams(dim, dim, S, 0)
    pc_sw = capi.BatchMatMulParams(ffn, dim, S, 0)
    pc_down = capi.BatchMatMulParams(dim, ffn, S, 0)
    fa = capi.FlashAttentionParams(128, H, S, 1.0 / math.sqrt(128.0))
    ad = p["adaln"]
    hp, ap, qp, atp, tp, fp = (x.data_ptr() for x in (hidden, buf_a, qkv, attn, t, f))

    def step():
        ck = capi.check
        ck(lib.llmr_batch_rmsnorm(h, hp, dim, p["attn_norm1"], ad, None, ap, F32, dim, dim, S, ctypes.c_float(eps)))
        ck(lib.llmr_batch_matmul_pc(h, p["wqkv"], Q8, ap, F32, qp, ctypes.byref(pc_qkv)))
        ck(lib.llmr_qkv_heads(h, qp, 3 * dim, S, H, p["q_norm"], p["k_norm"], ctypes.c_float(eps), cos_t.data_ptr(),
                              sin_t.data_ptr(), qh.data_ptr(), kh.data_ptr(), vh.data_ptr(), F32, S, 0))
        ck(lib.llmr_flash_attention_pc(h, qh.data_ptr(), kh.data_ptr(), vh.data_ptr(), F32, atp, ctypes.byref(fa)))
        ck(lib.llmr_batch_matmul_pc(h, p["wo"], Q8, atp, F32, tp, ctypes.byref(pc_o)))
        ck(lib.llmr_gated_residual(h, hp, dim, tp, dim, p["attn_norm2"], ad + 4 * dim, capi.GATE_TANH, dim, S,
                                   ctypes.c_float(eps)))
        ck(lib.llmr_batch_rmsnorm(h, hp, dim, p["ffn_norm1"], ad + 8 * dim, None, ap, F32, dim, dim, S,
                                  ctypes.c_float(eps)))
        ck(lib.llmr_batch_matmul_swiglu_pc(h, p["w_gate"], p["w_up"], Q8, ap, F32, fp, ctypes.byref(pc_sw)))
        ck(lib.llmr_batch_matmul_pc(h, p["w_down"], Q8, fp, F32, tp, ctypes.byref(pc_down)))
        ck(lib.llmr_gated_residual(h, hp, dim, tp, dim, p["ffn_norm2"], ad + 12 * dim, capi.GATE_TANH, dim, S,
                                   ctypes.c_float(eps)))

    flops = 2.0 * S * dim * (3 * dim + dim + 2 * ffn + ffn) + a.flops
    cfg = {"workload": "zimage_block_c3", "hidden": dim, "heads": H, "head_dim": 128, "ffn": ffn, "seq_len": S,
           "weights": "Q8_0", "activations": "f32 (every buffer, as the reference's)",
           "calls": "tests/c/zimage_layer.c order: rmsnorm, batch_matmul_pc (QKV), qkv_heads (f32), "
           "flash_attention_pc (f32), batch_matmul_pc (O), gated_residual, rmsnorm, batch_matmul_swiglu_pc, "
           "batch_matmul_pc (down), gated_residual"}
    return step, flops, None, cfg, "f32"


def setup_flux_step(dev, mlp_act: str = "gelu"):
    """One denoising forward of the Flux-dev-shaped DiT (19 double + 38 single
    blocks, hidden 3072, 24 heads, MLP 12288, Q4_K weights generated on the
    device, 4096 image tokens from 16x128x128 latents + 512 text tokens).
    mlp_act "swiglu": the reference's own Flux.2 MLP form (linear1 [3 d +
    2 m, d], MLP in-projections [2 m, d], silu(gate) * up in the GEMMs'
    epilogue)."""
    import dataclasses

    import torch
    from llmr_amd import dit, synth, workloads
    cfg_m = dataclasses.replace(dit.FLUX_DEV, mlp_act=mlp_act)
    glob, doubles, singles = dit.flux_weights(cfg_m, device=dev)
    model = dit.FluxDiT(cfg_m, glob, doubles, singles, act_dtype=torch.bfloat16, device=dev)
    lat = torch.from_numpy(synth.normal(workloads.SEED, 30, cfg_m.latent_ch * cfg_m.latent_h * cfg_m.latent_w)
                           .reshape(cfg_m.latent_ch, cfg_m.latent_h, cfg_m.latent_w)).to(dev)
    txt = torch.from_numpy(synth.normal(workloads.SEED, 31, cfg_m.n_txt * cfg_m.text_dim)
                           .reshape(cfg_m.n_txt, cfg_m.text_dim)).to(dev).to(torch.bfloat16)

    def step():
        model.forward(lat, txt, 0.5)

    cfg = {"workload": "flux_step" if mlp_act == "gelu" else "flux2_step", "double_blocks": cfg_m.n_double,
           "single_blocks": cfg_m.n_single, "hidden": cfg_m.dim, "heads": cfg_m.n_heads, "mlp": cfg_m.mlp,
           "img_tokens": cfg_m.n_img, "txt_tokens": cfg_m.n_txt, "weights": "Q4_K (img_in Q8_0)",
           "activations": "bf16", "timestep": 0.5,
           "mlp_act": "gelu-tanh" if mlp_act == "gelu" else "swiglu (silu(gate) * up)", "modulation": "per block"}
    return step, cfg_m.gemm_flops(), None, cfg, "bf16"


MODEL_SETUPS = {"zimage_block": setup_zimage_block, "zimage_block_c3": setup_zimage_block_c3,
                "flux_step": setup_flux_step,
                "flux2_step": lambda dev: setup_flux_step(dev, "swiglu")}


def gemm_kernel_name(name: str, num_cus: int) -> str:
    """The kernels the library's dispatch runs for a GEMM workload (the one
    that dominates first): the two-pass path (weight image, then the all-DMA
    persistent GEMM) from 2048 tokens with at least half the CUs' worth of
    256 x 256 tiles; the one-pass persistent kernels below 2048 tokens; up to
    256 tokens the few-token kernel (one launch) when there are at least half
    the CUs' worth of 32 x 96 tiles, else the split-K skinny kernel; else the
    4-wave tiled kernel."""
    from llmr_amd import gguf, workloads
    g = workloads.GEMMS[name]
    tiles = ((g.M + 255) // 256) * ((g.N + 255) // 256)
    if g.wtype == gguf.GGML_Q8_0 and g.K % 64:
        return "gemm_q_generic"
    if g.wtype == gguf.GGML_Q4_K and g.M <= 4:
        return "gemv_q4k"
    f32 = g.xtype == gguf.GGML_F32
    cvt = "f32->bf16" if g.wtype == gguf.GGML_Q4_K else "f32->f16"
    if g.K % 64 == 0 and g.N % 4 == 0 and 2 * tiles >= num_cus:
        if g.M >= 2048:
            return "gemm_w16_persist + w16_image_kernel" + (f" + {cvt} conversion" if f32 else "")
        return (f"{cvt} conversion + " if f32 else "") + ("gemm_q_persist8" if g.wtype == gguf.GGML_Q8_0
                                                          else "gemm_q_persist")
    few_tiles = ((g.M + 31) // 32) * ((g.N + 95) // 96)
    if g.M <= 256 and g.K % 64 == 0 and 2 * few_tiles >= num_cus:
        return "gemm_q_few"
    if g.M <= 256 and g.K % 64 == 0 and g.N % 4 == 0:
        return "gemm_q_skinny + splitk_reduce_kernel" + (" + skinny_pack_kernel" if f32 else "")
    return "gemm_q_mfma"


def kernel_name(name: str, num_cus: int) -> str:
    """The kernels a kernel-level workload runs (the dominant one first)."""
    from llmr_amd import workloads
    if name == "flux_attention":
        return "flash_attn_fwd64_w8"
    if name == "flux_attention_f32":
        return "flash_attn_fwd64_w8 + kv_to_f16_kernel"
    if name == "flux_linear1_lora":
        return "gemm_w16_persist + w16_image_kernel (LoRA merged)"
    if name in workloads.SWIGLUS:
        return "gemm_w16_persist (SwiGLU) + w16_image_kernel"
    return gemm_kernel_name(name, num_cus)


def measure(dev, name, steps, warmup, cold: bool = False):
    from llmr_amd import workloads
    if name in ("flux_attention", "flux_attention_f32"):
        step, flops, nbytes, cfg, dtype = setup_attention(dev, f32=name.endswith("_f32"))
    elif name in MODEL_SETUPS:
        step, flops, nbytes, cfg, dtype = MODEL_SETUPS[name](dev)
    elif name in workloads.SWIGLUS:
        step, flops, nbytes, cfg, dtype = setup_swiglu(dev, name)
    elif name == "lora_flux_linear1":
        step, flops, nbytes, cfg, dtype = setup_lora(dev)
    elif name == "flux_linear1_lora":
        step, flops, nbytes, cfg, dtype = setup_gemm_lora(dev)
    else:
        step, flops, nbytes, cfg, dtype = setup_gemm(dev, name)
    cold_ms = None
    if cold:  # W warmup + K timed steps straight after set-up, before the device warm-up
        cold_ms = _time_steps(step, steps, warmup)[0] / steps
    _device_warmup(step)
    total_ms, per = _time_steps(step, steps, warmup, per_step=name in MODEL_SETUPS)
    ms = total_ms / steps
    med = sorted(per)[len(per) // 2] if per else ms
    tflops = flops / (ms * 1e-3) / 1e12
    return {"name": name, "ms": ms, "median_ms": med, "tflops": tflops, "flops": flops,
            "bytes": nbytes, "cfg": cfg, "dtype": dtype, "cold_ms": cold_ms}


def library_baselines(steps: int, warmup: int) -> int:
    """The vendor libraries on the same shapes, timed as the workloads are
    (device warm-up, W warmup and K timed steps between two HIP events),
    each beside this library's own call in the same process: hipBLASLt
    (torch.mm) on plain bf16 operands (no dequantization) with f32 and with
    bf16 output, against the Q4_K / Q8_0 dequant-GEMM with its f32 output;
    PyTorch's scaled_dot_product_attention (flash backend) against the flash
    attention call. One JSON line per shape."""
    import torch
    import torch.nn.functional as F
    from llmr_amd import workloads
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(42)
    for name in ("flux_linear1", "flux_linear2", "zimage_qkv"):
        g = workloads.GEMMS[name]
        r = measure(dev, name, steps, warmup)
        x = torch.randn(g.M, g.K, dtype=torch.bfloat16, device=dev, generator=gen)
        wt = (torch.randn(g.N, g.K, dtype=torch.bfloat16, device=dev, generator=gen) * 0.02).t()
        flops = 2.0 * g.M * g.N * g.K
        line = {"shape": name, "M": g.M, "N": g.N, "K": g.K}
        for key, fn in (("hipblaslt_bf16_to_f32", lambda: torch.mm(x, wt, out_dtype=torch.float32)),
                        ("hipblaslt_bf16_to_bf16", lambda: torch.mm(x, wt))):
            _device_warmup(fn)
            ms = _time_steps(fn, steps, warmup)[0] / steps
            line[key] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
        del x, wt
        line["llmr_" + r["dtype"]] = {"ms": round(r["ms"], 4), "tflops": round(r["tflops"], 1),
                                      "weight": r["cfg"].get("weight"), "output": "f32"}
        print(json.dumps(line), flush=True)
    a = workloads.FLUX_ATTENTION
    r = measure(dev, "flux_attention", steps, warmup)
    q, k, v = (torch.randn(1, a.H, a.S, a.D, dtype=torch.float16, device=dev, generator=gen) for _ in range(3))
    from torch.nn.attention import SDPBackend, sdpa_kernel
    flops = 4.0 * a.H * a.S * a.S * a.D
    line = {"shape": "flux_attention", "H": a.H, "S": a.S, "D": a.D}
    with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
        fn = lambda: F.scaled_dot_product_attention(q, k, v)
        _device_warmup(fn)
        ms = _time_steps(fn, steps, warmup)[0] / steps
    line["torch_sdpa_flash_f16"] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
    line["llmr_f16"] = {"ms": round(r["ms"], 4), "tflops": round(r["tflops"], 1)}
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(name: str, budget_s: float = 10.0):
    """The oracle (the C restatement, OpenMP on the host cores) on a bounded
    sample of the same workload: whole heads (attention) or token blocks
    (GEMM) until about `budget_s` seconds of oracle time have been spent."""
    import numpy as np
    from oracle import oracle as orc
    from llmr_amd import workloads
    orc.lib()
    dt = 0.0
    flops = 0.0
    if name == "flux_attention":
        a = workloads.FLUX_ATTENTION
        h = 0
        while h < a.H and dt < budget_s:
            q, k, v = (t.astype(np.float32) for t in workloads.attention_inputs(a, heads=(h, h + 1)))
            t0 = time.perf_counter()
            orc.flash_attention(q, k, v, 1.0 / math.sqrt(a.D))
            dt += time.perf_counter() - t0
            flops += 4.0 * a.S * a.S * a.D
            h += 1
        sample = f"{h} of {a.H} heads, all {a.S} queries x {a.S} keys"
    else:
        g = workloads.GEMMS[name]
        blk = workloads.gemm_weight_blocks(g)
        x = workloads.gemm_activations_f32(g)
        m = 0
        while m < g.M and dt < budget_s:
            rows = np.arange(m, min(m + 16, g.M), dtype=np.uint32)
            t0 = time.perf_counter()
            orc.batch_matmul(blk, g.wtype, x, g.N, g.K, g.M, 0, rows=rows)
            dt += time.perf_counter() - t0
            flops += 2.0 * len(rows) * g.N * g.K
            m += len(rows)
        sample = f"{m} of {g.M} tokens, all {g.N} outputs"
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": orc.num_threads(),
            "kind": "port", "sample": sample + f", {dt:.1f} s of oracle time"}


def copy_calibration(steps: int, warmup: int) -> int:
    """A plain device-to-device copy of 1 GiB (reads 1 GiB, writes 1 GiB): the
    known-size kernel the HBM traffic counters are scaled by."""
    import torch
    n = 1 << 28
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    total_ms, _ = _time_steps(lambda: b.copy_(a), steps, warmup)
    ms = total_ms / steps
    print(json.dumps({"calibration": "hbm_copy", "bytes_read": 4 * n, "bytes_written": 4 * n,
                      "ms": round(ms, 4), "gbs": round(8 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="flux_attention")
    ap.add_argument("--components",
                    default="flux_linear1,flux_linear2,q8_linear,zimage_qkv,zimage_swiglu,flux_linear1_f32,"
                            "flux_linear2_f32,flux_attention_f32,lora_flux_linear1,flux_linear1_lora,zimage_block,"
                            "zimage_block_c3,flux_step,"
                            "flux2_step")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--hbm-copy-calibration", action="store_true",
                    help="time a plain 1 GiB device copy (reference for the FETCH_SIZE/WRITE_SIZE counters)")
    ap.add_argument("--library-baselines", action="store_true",
                    help="time hipBLASLt GEMMs and PyTorch's flash attention on the same shapes beside this library")
    args = ap.parse_args()
    if args.hbm_copy_calibration:
        return copy_calibration(args.steps, args.warmup)
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
              "(the hot path is single-GPU; sharding is design-only)", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    from llmr_amd import capi
    capi.lib()  # fail loudly if the HIP library is missing
    if args.library_baselines:
        return library_baselines(args.steps, args.warmup)

    main_r = measure(dev, args.workload, args.steps, args.warmup, cold=True)
    comps = {}
    for c in [c for c in args.components.split(",") if c and c != args.workload]:
        if c in MODEL_SETUPS:  # whole blocks / steps: fewer, longer steps
            r = measure(dev, c, max(3, args.steps // 10), max(1, args.warmup // 2))
            comps[c] = {"ms_per_step": round(r["ms"], 3), "median_ms": round(r["median_ms"], 3),
                        "tflops_gemm_attention": round(r["tflops"], 2),
                        "frac_of_peak": round(r["tflops"] / PEAK_TFLOPS, 4), "config": r["cfg"]}
        else:
            r = measure(dev, c, max(5, args.steps // 2), args.warmup)
            comps[c] = {"tflops": round(r["tflops"], 2), "ms_per_call": round(r["ms"], 4),
                        "frac_of_peak": round(r["tflops"] / PEAK_TFLOPS, 4),
                        "hbm_gbs_algorithmic": round(r["bytes"] / (r["ms"] * 1e-3) / 1e9, 1),
                        "config": r["cfg"]}
        print(f"# {c}: {json.dumps(comps[c])}", file=sys.stderr, flush=True)

    ach = main_r["tflops"]
    if args.workload == "lora_flux_linear1":  # bandwidth-bound: priced against HBM
        gbs = main_r["bytes"] / (main_r["ms"] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": _traffic(args.workload),
                "kernel": "lora_down_kernel + lora_up_reg_kernel", "algorithmic_bytes": main_r["bytes"]}
    elif args.workload in MODEL_SETUPS:  # a composed block / step: many kernels, no single roofline
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_TFLOPS, 4), "traffic": None,
                "kernel": "composite (GEMM + attention + glue; GEMM and attention flops counted)"}
    else:
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_TFLOPS, 4), "traffic": _traffic(args.workload),
                "kernel": kernel_name(args.workload, torch.cuda.get_device_properties(dev).multi_processor_count),
                "algorithmic_bytes": main_r["bytes"],
                "hbm_frac_algorithmic": round(main_r["bytes"] / (main_r["ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    line = {
        "metric": METRIC,
        "value": round(ach, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_r["ms"], 5),
        # untimed GPU time of back-to-back steps before the W warmup steps,
        # and the K steps timed straight after set-up without it
        "device_warmup_ms": DEVICE_WARMUP_MS,
        "cold_ms_per_step": round(main_r["cold_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": main_r["dtype"],
        "data": "synthetic (SplitMix64/Box-Muller, seed 42; weights N(0,0.02) quantized, activations N(0,1))",
        "config": main_r["cfg"],
        "roofline": roof,
        "components": comps,
    }
    if not args.no_cpu_baseline and args.workload not in MODEL_SETUPS and args.workload != "lora_flux_linear1":
        line["cpu_baseline"] = cpu_baseline(args.workload)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
