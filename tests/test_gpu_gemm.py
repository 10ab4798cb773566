"""GPU dequant-GEMM vs the oracle (relative L2 <= 1e-2, the bar for GEMM
outputs; the oracle restates batch_matmul_q8 / batch_matmul_q4k)."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-2  # relative L2 vs the reference arithmetic (bf16/fp16 operands, f32 accumulate)


def _torch_x(x_f32, xtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x_f32))
    if xtype == 1:
        t = t.to(torch.float16)
    elif xtype == 30:
        t = t.to(torch.bfloat16)
    return t.to(dev)


def _x_as_f32(x_t):
    import torch
    return x_t.to(torch.float32).cpu().numpy()


def _run(dev, blk, wtype, x_f32, xtype, N, row_offset=0):
    import torch
    from llmr_amd import ops
    w = torch.from_numpy(blk).to(dev)
    xt = _torch_x(x_f32, xtype, dev)
    y = ops.batch_matmul(w, wtype, xt, N, row_offset=row_offset)
    torch.cuda.synchronize()
    return y.cpu().numpy(), _x_as_f32(xt)


CASES = [
    # (wtype, M, N, K, xtype, row_offset)
    (8, 256, 3072, 3072, 0, 0),      # the single Q8_0 linear, f32 activations, full size
    (8, 100, 200, 512, 30, 0),       # ragged M/N, bf16
    (8, 65, 130, 256, 1, 64),        # f16, row_offset into a fused weight
    (8, 7, 33, 96, 0, 3),            # K % 64 == 32: generic kernel; N not a multiple of 4
    (8, 1, 64, 64, 30, 0),           # one token
    (8, 300, 520, 1024, 30, 8),      # 128x128 tiles, ragged
    (12, 77, 130, 512, 0, 0),        # Q4_K f32
    (12, 129, 256, 1024, 30, 256),   # Q4_K bf16 with row_offset
    (12, 513, 1032, 768, 1, 0),      # Q4_K f16, ragged
    (12, 1, 17, 256, 30, 1),         # one token, odd N (small-M Q4_K kernel)
    (12, 3, 1000, 768, 1, 4),        # small-M Q4_K kernel, f16, row_offset
    (12, 4, 130, 512, 30, 0),        # small-M Q4_K kernel at its largest M
    (12, 5, 72, 512, 30, 0),         # one token more: the tiled kernel again
    # few tokens with at least half the CUs' worth of 32 x 96 tiles: the
    # few-token kernel (one launch, the waves of a workgroup split K)
    (8, 250, 3001, 3264, 30, 5),     # ragged M, odd N, 51 stages (not a multiple of the 8 waves), bf16
    (12, 256, 2048, 2560, 0, 256),   # Q4_K f32 (bf16 operands), row_offset
    (8, 129, 4000, 1024, 1, 0),      # one token in the last token tile, f16
    (12, 64, 12288, 512, 1, 0),      # Q4_K f16, two token tiles
    (12, 256, 3072, 3072, 30, 0),    # Q4_K bf16 at the single-linear size
    # few tokens over few features, N % 4 == 0: the skinny kernel (all tokens x
    # 64 features per workgroup, K split across workgroups)
    (8, 200, 1000, 768, 30, 8),      # ragged M and N, bf16, row_offset
    (8, 33, 64, 4096, 0, 0),         # one feature tile: 16 K splits, f32
    (12, 250, 3072, 3072, 1, 0),     # Q4_K f16 at the single-linear size
    (12, 256, 21504, 1024, 30, 0),   # 336 feature tiles: no split
    (8, 17, 128, 192, 1, 0),         # three stages: one split, short pipeline
    (12, 100, 256, 1024, 0, 256),    # Q4_K, f32 activations packed to fp16, row_offset
]


@pytest.mark.parametrize("M,N,K,row_offset", [(1, 18432, 3072, 0), (1, 3072, 256, 0), (4, 264, 4096, 16)])
def test_small_m_q4k_f32_matches_reference_arithmetic(orc, dev, M, N, K, row_offset):
    """M <= 4 Q4_K launches keep the activations in f32 and sum the
    f32 products of batch_matmul_q4k's dequantized weights (per sub-block as
    d*sc * sum q x - dmin*mn * sum x): only the rounding order differs from
    the oracle, far inside the GEMM bar (the modulation-projection shape
    first)."""
    from llmr_amd import gguf, synth
    blk = gguf.quantize(synth.normal(21, 2, (N + row_offset) * K, 0.02), 12)
    x = synth.normal(21, 1, M * K).reshape(M, K)
    y, xr = _run(dev, blk, 12, x, 0, N, row_offset)
    ref = orc.batch_matmul(blk, 12, xr, N, K, M, row_offset)
    err = rel_l2(y, ref)
    print(f"small-M Q4_K M={M} N={N} K={K}: rel_l2={err:.3e}")
    assert err <= 1e-5


@pytest.mark.parametrize("wtype,M,N,K,xtype,row_offset", CASES)
def test_gemm_parity(orc, dev, wtype, M, N, K, xtype, row_offset):
    from llmr_amd import gguf, synth
    rows = N + row_offset + 5
    w32 = synth.normal(3, 2, rows * K, 0.02)
    blk = gguf.quantize(w32, wtype)
    x = synth.normal(3, 1, M * K).reshape(M, K)
    y, xr = _run(dev, blk, wtype, x, xtype, N, row_offset)
    ref = orc.batch_matmul(blk, wtype, xr, N, K, M, row_offset)
    err = rel_l2(y, ref)
    print(f"wtype={wtype} M={M} N={N} K={K} xtype={xtype} off={row_offset}: rel_l2={err:.3e}")
    assert np.all(np.isfinite(y))
    assert err <= TOL


@pytest.mark.parametrize("wtype", [8, 12])
def test_row_offset_slices_equal_fused_call(dev, wtype):
    """Slot calls (row_offset = 0, n, 2n) reproduce the columns of one fused call."""
    from llmr_amd import gguf, synth
    M, n, K = 96, 256, 512
    blk = gguf.quantize(synth.normal(5, 2, 3 * n * K, 0.02), wtype)
    x = synth.normal(5, 1, M * K).reshape(M, K)
    full, _ = _run(dev, blk, wtype, x, 30, 3 * n)
    for s in range(3):
        part, _ = _run(dev, blk, wtype, x, 30, n, row_offset=s * n)
        assert np.array_equal(part, full[:, s * n:(s + 1) * n])


def test_identity_weights_select_columns(dev):
    """W[n, k] = [k == n] (Q8_0 scale 1/127, q = 127): each output is one product."""
    from llmr_amd import gguf
    M, N, K = 64, 128, 128
    w = np.zeros((N, K), np.float32)
    w[np.arange(N), np.arange(N)] = 1.0
    blk = gguf.quantize_q8_0(w)
    x = (np.arange(M * K, dtype=np.float32).reshape(M, K) % 97 - 48) / 16.0  # exact in fp16
    y, _ = _run(dev, blk, 8, x, 0, N)
    d16 = np.float16(1.0 / 127.0)
    c = np.float32(np.float16(d16 * np.float16(127)))
    assert np.array_equal(y, x[:, :N] * c)


def test_zero_and_nonfinite_scales(orc, dev):
    """All-zero blocks give exact zeros; an Inf scale block poisons only its own outputs."""
    from llmr_amd import gguf, synth
    M, N, K = 32, 64, 256
    blk = gguf.quantize_q8_0(synth.normal(9, 2, N * K, 0.02)).reshape(N, K // 32, 34).copy()
    blk[5] = 0                                  # row 5: all-zero blocks
    blk[9, 2, 0:2] = np.array([0x7C00], np.uint16).view(np.uint8)  # row 9 block 2: scale +Inf
    x = synth.normal(9, 1, M * K).reshape(M, K)
    y, xr = _run(dev, blk.reshape(-1), 8, x, 0, N)
    assert np.all(y[:, 5] == 0)
    assert not np.any(np.isfinite(y[:, 9]))
    mask = np.ones(N, bool)
    mask[[5, 9]] = False
    ref = orc.batch_matmul(blk.reshape(-1), 8, xr, N, K, M, 0)
    assert rel_l2(y[:, mask], ref[:, mask]) <= TOL


# Shapes with at least 128 tiles of 256 x 256 take the persistent kernel
# (16-bit activations, N % 4 == 0): ragged M and N, more tiles than CUs (two
# per workgroup, some workgroups splitting their first tile in two K pieces),
# stage counts that are not a multiple of 6 (zero-padded stages), row_offset
# into a fused weight, both activation types.
PERSIST_CASES = [
    # (wtype, M, N, K, xtype, row_offset)
    (12, 4100, 4100, 768, 30, 0),
    (8, 4100, 4100, 768, 30, 16),
    (8, 4100, 4100, 320, 1, 0),
    (12, 2000, 4352, 1024, 1, 256),
    (8, 2560, 3332, 640, 1, 4),
    (8, 4096, 3072, 64, 30, 0),   # Flux img_in: one real K stage of six
    # last rounds of 216 and 136 tiles too short in K to split (2-3 groups of
    # 6 stages per tile): they stay whole
    (12, 4608, 3072, 1024, 30, 0),
    (8, 4608, 3072, 640, 1, 0),      # Q8_0 f16, 10 of 12 stages real
    (12, 4608, 9216, 768, 30, 16),   # 648 tiles: 2 whole rounds + 136
    # f32 activations rounded to fp16 in the workspace first: from 2048
    # tokens the two-pass path, below it the fused kernel
    (12, 4100, 4100, 768, 0, 0),
    (8, 2560, 3332, 640, 0, 4),
    (8, 1024, 8192, 512, 0, 0),
    (12, 1500, 5376, 512, 0, 256),
]


@pytest.mark.parametrize("wtype,M,N,K,xtype,row_offset", PERSIST_CASES)
def test_persistent_kernel_sampled_rows(orc, dev, wtype, M, N, K, xtype, row_offset):
    import torch
    from llmr_amd import gguf, ops, synth
    blk = gguf.quantize(synth.normal(13, 2, (N + row_offset + 3) * K, 0.02), wtype)
    x = synth.normal(13, 1, M * K).reshape(M, K)
    w = torch.from_numpy(blk).to(dev)
    xt = _torch_x(x, xtype, dev)
    y = ops.batch_matmul(w, wtype, xt, N, row_offset=row_offset)
    torch.cuda.synchronize()
    rows = np.unique(np.array([0, 1, 31, 32, 255, 256, 511, 1024 + 7, M // 2, M - 257, M - 256, M - 2, M - 1],
                              np.int64).clip(0, M - 1)).astype(np.uint32)  # every sampled row < M
    ref = orc.batch_matmul(blk, wtype, _x_as_f32(xt), N, K, M, row_offset, rows=rows)
    got = y[torch.from_numpy(rows.astype(np.int64)).to(dev)].cpu().numpy()
    err = rel_l2(got, ref)
    print(f"persistent wtype={wtype} M={M} N={N} K={K} xtype={xtype}: sampled rel_l2={err:.3e}")
    assert np.all(np.isfinite(got))
    assert err <= TOL
    # every column block of every sampled row is right (no tile left unwritten)
    for c0 in range(0, N, 256):
        assert rel_l2(got[:, c0:c0 + 256], ref[:, c0:c0 + 256]) <= 2 * TOL


# Persistent launches checked tile by tile, with part-filled last rounds of
# 256 x 256 tiles (on 256 CUs) and ragged edges.
TILE_CASES = [
    # (wtype, M, N, K, xtype, row_offset)
    (12, 4608, 3072, 3072, 30, 0),   # 216 tiles: one part-filled round
    (12, 4608, 9216, 3072, 30, 0),   # 648 tiles: 2 whole rounds + 136
    (12, 4608, 12288, 3072, 30, 0),  # 864 tiles: 3 whole rounds + 96
    (8, 4500, 3000, 3072, 1, 16),    # Q8_0 f16, ragged edges, row_offset
    (12, 2048, 4096, 3072, 1, 0),    # 128 tiles, fewer than the CUs
    (8, 2048, 4096, 1088, 30, 0),    # 17 real stages of 18
]


def _weights(dev, wtype, rows, K, seed):
    import torch
    from llmr_amd import glue, gguf, synth
    if wtype == 12:
        return glue.synth_q4k(rows, K, seed, device=dev)
    return torch.from_numpy(gguf.quantize(synth.normal(seed, 2, rows * K, 0.02), wtype)).to(dev)


@pytest.mark.parametrize("wtype,M,N,K,xtype,row_offset", TILE_CASES)
def test_persistent_every_tile(dev, wtype, M, N, K, xtype, row_offset):
    """Every 256 x 256 tile of a persistent launch against an f32 product of
    the dequantized weight (rel L2 per tile: a tile left unwritten or summed
    over the wrong K range fails); the same launch repeated after another
    launch gives the same bits."""
    import torch
    from llmr_amd import ops
    w = _weights(dev, wtype, N + row_offset, K, 70 + wtype)
    g = torch.Generator(device="cpu").manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(torch.float16 if xtype == 1 else torch.bfloat16).to(dev)
    y = ops.batch_matmul(w, wtype, x, N, row_offset=row_offset)
    ref = x.float() @ ops.dequant(w, wtype, N, K, row_offset).t()
    torch.cuda.synchronize()
    tm, tn = (M + 255) // 256, (N + 255) // 256
    pad = (0, tn * 256 - N, 0, tm * 256 - M)
    d2 = torch.nn.functional.pad((y - ref).double() ** 2, pad).view(tm, 256, tn, 256).sum((1, 3))
    r2 = torch.nn.functional.pad(ref.double() ** 2, pad).view(tm, 256, tn, 256).sum((1, 3))
    err = (d2 / r2).sqrt()
    print(f"every tile wtype={wtype} M={M} N={N} K={K}: worst tile rel_l2={float(err.max()):.3e}")
    assert bool(torch.isfinite(y).all())
    assert float(err.max()) <= TOL
    other = ops.batch_matmul(w, wtype, x[:2048].contiguous(), 4096 if N >= 4096 else N)
    y2 = ops.batch_matmul(w, wtype, x, N, row_offset=row_offset)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(other).all())
    assert torch.equal(y, y2)


@pytest.mark.parametrize("name", ["flux_linear1", "flux_linear2", "zimage_qkv"])
def test_full_size_sampled_rows(orc, dev, name):
    """Full-size launches; the oracle checks a sample of tokens (every column)."""
    import torch
    from llmr_amd import ops, workloads
    g = workloads.GEMMS[name]
    blk = workloads.gemm_weight_blocks(g)
    x = workloads.gemm_activations_f32(g)
    w = torch.from_numpy(blk).to(dev)
    xt = _torch_x(x, g.xtype, dev)
    y = ops.batch_matmul(w, g.wtype, xt, g.N)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 1023, g.M // 2 + 3, g.M - 2, g.M - 1], np.uint32)
    ref = orc.batch_matmul(blk, g.wtype, x, g.N, g.K, g.M, 0, rows=rows)
    got = y[torch.from_numpy(rows.astype(np.int64)).to(dev)].cpu().numpy()
    err = rel_l2(got, ref)
    print(f"{name}: sampled rel_l2={err:.3e}")
    assert err <= TOL
    # row independence: the same token computed alone (a one-token launch,
    # which takes the small-tile kernel) agrees with the oracle and with its
    # row of the full launch to within both kernels' operand rounding
    m = int(rows[5])
    y1 = ops.batch_matmul(w, g.wtype, xt[m:m + 1].contiguous(), g.N)
    torch.cuda.synchronize()
    y1 = y1.cpu().numpy()[0]
    assert rel_l2(y1, ref[5]) <= TOL
    assert rel_l2(y1, y[m].cpu().numpy()) <= 2 * TOL


SWIGLU_CASES = [
    # (M, N, K, xtype)
    (100, 256, 512, 30),   # bf16, fused kernel, ragged M
    (300, 520, 1024, 1),   # f16, fused, N not a multiple of 128
    (65, 260, 256, 0),     # f32 activations: rounded to bf16, then fused
    (7, 34, 96, 30),       # N % 4 != 0 and K % 64 == 32: two GEMMs + elementwise SwiGLU
    (1, 64, 64, 30),       # one token
    (513, 1032, 768, 30),  # more tiles than workgroups in one round on small GPUs
]


@pytest.mark.parametrize("M,N,K,xtype", SWIGLU_CASES)
def test_swiglu_parity(orc, dev, M, N, K, xtype):
    from llmr_amd import gguf, ops, synth
    wg = gguf.quantize_q8_0(synth.normal(21, 1, N * K, 0.05))
    wu = gguf.quantize_q8_0(synth.normal(21, 2, N * K, 0.05))
    x = synth.normal(21, 3, M * K).reshape(M, K)
    import torch
    xt = _torch_x(x, xtype, dev)
    y = ops.batch_matmul_swiglu(torch.from_numpy(wg).to(dev), torch.from_numpy(wu).to(dev), xt, N)
    torch.cuda.synchronize()
    ref = orc.batch_matmul_swiglu_q8(wg, wu, _x_as_f32(xt), N, K, M)
    err = rel_l2(y.cpu().numpy(), ref)
    print(f"swiglu M={M} N={N} K={K} xtype={xtype}: rel_l2={err:.3e}")
    assert np.all(np.isfinite(y.cpu().numpy()))
    assert err <= TOL
    # gate and up are not interchangeable: the swapped product is far off
    swapped = orc.batch_matmul_swiglu_q8(wu, wg, _x_as_f32(xt), N, K, M)
    assert rel_l2(y.cpu().numpy(), swapped) > 10 * TOL


def test_swiglu_matches_two_gemms(dev):
    """The fused kernel equals silu(gate GEMM) * up GEMM from the plain entry point
    (f16 activations: the same fp16 operands on both paths) to f32 rounding."""
    import torch
    from llmr_amd import gguf, ops, synth
    M, N, K = 512, 512, 1024
    wg = torch.from_numpy(gguf.quantize_q8_0(synth.normal(22, 1, N * K, 0.05))).to(dev)
    wu = torch.from_numpy(gguf.quantize_q8_0(synth.normal(22, 2, N * K, 0.05))).to(dev)
    x = _torch_x(synth.normal(22, 3, M * K).reshape(M, K), 1, dev)
    y = ops.batch_matmul_swiglu(wg, wu, x, N)
    g = ops.batch_matmul(wg, 8, x, N)
    u = ops.batch_matmul(wu, 8, x, N)
    torch.cuda.synchronize()
    ref = (g / (1 + torch.exp(-g)) * u).cpu().numpy()
    assert rel_l2(y.cpu().numpy(), ref) < 1e-5


def test_swiglu_pc_rejects_row_offset(dev):
    import ctypes
    import torch
    from llmr_amd import capi, gguf, ops, synth
    N, K, M = 64, 64, 4
    w = torch.from_numpy(gguf.quantize_q8_0(synth.normal(23, 1, N * K, 0.05))).to(dev)
    x = torch.zeros((M, K), dtype=torch.bfloat16, device=dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    g = ops.default_graph()
    g.bind_stream()
    pc = capi.BatchMatMulParams(N, K, M, 1)
    rc = capi.lib().llmr_batch_matmul_swiglu_pc(g.ctx.handle, w.data_ptr(), w.data_ptr(), 8, x.data_ptr(), 30,
                                                y.data_ptr(), ctypes.byref(pc))
    assert rc == capi.LLMR_ERR_INVALID_ARG
    rc = capi.lib().llmr_batch_matmul_swiglu(g.ctx.handle, w.data_ptr(), w.data_ptr(), 12, x.data_ptr(), 30,
                                             y.data_ptr(), N, K, M)
    assert rc == capi.LLMR_ERR_UNSUPPORTED


def test_swiglu_full_size_sampled(orc, dev):
    """The Z-Image FFN in-projection at full size; sampled tokens vs the oracle."""
    import torch
    from llmr_amd import ops, workloads
    g = workloads.ZIMAGE_SWIGLU
    wg_np = workloads.gemm_weight_blocks(g)
    wg = torch.from_numpy(wg_np).to(dev)
    wu_np = workloads.swiglu_up_blocks(g)
    wu = torch.from_numpy(wu_np).to(dev)
    x = workloads.gemm_activations_f32(g)
    xt = _torch_x(x, g.xtype, dev)
    y = ops.batch_matmul_swiglu(wg, wu, xt, g.N)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 2049, g.M - 2, g.M - 1], np.uint32)
    ref = orc.batch_matmul_swiglu_q8(wg_np, wu_np, x, g.N, g.K, g.M, rows=rows)
    got = y[torch.from_numpy(rows.astype(np.int64)).to(dev)].cpu().numpy()
    err = rel_l2(got, ref)
    print(f"zimage_swiglu: sampled rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M,N,K", [(64, 128, 512), (2304, 2304, 512), (2304, 4096, 512)])
def test_bf16_activations_beyond_fp16_range(orc, dev, M, N, K):
    """bf16 activations of magnitude ~1e5 (past fp16's 65504) stay finite: every
    kernel uses bf16 operands for bf16 inputs (64 tokens: the few-token kernel;
    2304 x 2304: the 4-wave tiled kernel; 2304 x 4096: the two-pass path), where
    Q4_K weights become bf16 operands too."""
    import torch
    from llmr_amd import gguf, ops, synth
    blk = gguf.quantize_q4k(synth.normal(24, 1, N * K, 0.02))
    x = synth.normal(24, 2, M * K).reshape(M, K) * np.float32(1.0e5)
    y, xr = _run(dev, blk, 12, x, 30, N)
    rows = np.array([0, M // 2, M - 1], np.uint32)
    ref = orc.batch_matmul(blk, 12, xr, N, K, M, 0, rows=rows)
    assert np.all(np.isfinite(y))
    assert np.abs(xr).max() > 65504.0
    assert rel_l2(y[rows.astype(np.int64)], ref) <= TOL


@pytest.mark.parametrize("M,N,K,path", [(2048, 4096, 256, "two-pass"), (1024, 8192, 256, "persistent"),
                                        (256, 3072, 256, "few-token"), (100, 256, 512, "skinny"),
                                        (300, 520, 512, "tiled"), (3, 1000, 512, "gemv")])
def test_q4k_f32_activations_beyond_fp16_range(orc, dev, M, N, K, path):
    """f32 activations of magnitude ~1e5 against Q4_K weights stay finite and
    match the oracle on every kernel path: batch_matmul_q4k multiplies x in
    f32 (llm.slang:2300-2304), so its results are finite there; the MFMA
    paths round such x to bf16 (fp16 would overflow past 65504), the GEMV
    keeps f32."""
    from llmr_amd import gguf, synth
    blk = gguf.quantize_q4k(synth.normal(26, 1, N * K, 0.02))
    x = synth.normal(26, 2, M * K).reshape(M, K) * np.float32(1.0e5)
    print(f"Q4_K f32 x ~1e5 {path}: M={M} N={N} K={K}", flush=True)
    y, xr = _run(dev, blk, 12, x, 0, N)
    rows = np.unique(np.array([0, 1, M // 2, M - 1], np.uint32))
    ref = orc.batch_matmul(blk, 12, xr, N, K, M, 0, rows=rows)
    assert np.abs(xr).max() > 65504.0
    assert np.all(np.isfinite(y))
    err = rel_l2(y[rows.astype(np.int64)], ref)
    print(f"  rel_l2={err:.3e}")
    assert err <= TOL


# ---- llmr_batch_matmul_multi: grouped jobs and fused epilogues ----------------

def _multi_setup(dev, wtype, Ms, N, K, xtype, seed):
    import torch
    from llmr_amd import gguf, ops, synth
    blks, xs, wts = [], [], []
    for i, M in enumerate(Ms):
        blk = gguf.quantize(synth.normal(seed, 10 + i, (N + 8) * K, 0.02), wtype)
        x = synth.normal(seed, 20 + i, M * K).reshape(M, K)
        xt = _torch_x(x, xtype, dev)
        blks.append(blk)
        xs.append(xt)
        wts.append(ops.Tensor.quantized(torch.from_numpy(blk).to(dev), wtype, N + 8, K))
    return blks, xs, wts


def _sample_rows(M):
    return np.unique(np.array([0, 1, 63, 255, 256, M // 2, M - 2, M - 1], np.int64).clip(0, M - 1))


@pytest.mark.parametrize("wtype,xtype", [(12, 30), (8, 30), (12, 1)])
def test_multi_grouped_store_and_residual(orc, dev, wtype, xtype):
    """Two jobs (512 and 3584 tokens, own weights) in one persistent launch:
    a strided store, then a gated residual accumulate (one job without gate)."""
    import torch
    from llmr_amd import capi, ops
    Ms, N, K = (512, 3584), 2304, 512
    blks, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 31)
    g = ops.default_graph()
    out = torch.full((sum(Ms), N + 64), 5.0, dtype=torch.float32, device=dev)
    views = (out[:Ms[0], :N], out[Ms[0]:, :N])
    jobs = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), views[i], Ms[i], 4 * i) for i in range(2)]
    ops.dispatch_batch_matmul_multi(g, jobs, N, K)
    h0 = torch.randn(sum(Ms), N, device=dev)
    h = h0.clone()
    gate = torch.randn(N, device=dev)
    jobs = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), (h[:Ms[0]], h[Ms[0]:])[i], Ms[i], 4 * i,
                          gate if i == 0 else None) for i in range(2)]
    ops.dispatch_batch_matmul_multi(g, jobs, N, K, capi.EPI_GATED_RESIDUAL)
    torch.cuda.synchronize()
    assert (out[:, N:] == 5.0).all()  # columns past N untouched
    for i, M in enumerate(Ms):
        rows = _sample_rows(M)
        ref = orc.batch_matmul(blks[i], wtype, _x_as_f32(xs[i]), N, K, M, 4 * i, rows=rows)
        got = views[i][torch.from_numpy(rows).to(dev)].cpu().numpy()
        assert rel_l2(got, ref) <= TOL, (i, rel_l2(got, ref))
        hv = (h[:Ms[0]], h[Ms[0]:])[i][torch.from_numpy(rows).to(dev)].cpu().numpy()
        hb = (h0[:Ms[0]], h0[Ms[0]:])[i][torch.from_numpy(rows).to(dev)].cpu().numpy()
        gv = gate.cpu().numpy() if i == 0 else 1.0
        assert rel_l2(hv - hb, gv * ref) <= TOL, (i, rel_l2(hv - hb, gv * ref))


@pytest.mark.parametrize("xtype,pad", [(0, 0), (30, 0), (1, 0), (30, 40), (1, 40)])
def test_multi_gemv_group(orc, dev, xtype, pad):
    """Q4_K jobs of 1-4 tokens grouped in one call (the per-block modulation
    projections) run as one GEMV launch: every job equals its own
    single-job launch bit for bit and the oracle within the small-M bar
    (N = 300: a ragged last workgroup); rows past each job's M, and the
    columns between N and a row stride of N + pad, stay untouched."""
    import torch
    from llmr_amd import gguf, ops, synth
    N, K, Ms = 300, 512, (1, 3, 1, 4, 2, 1, 1)
    g = ops.default_graph()
    blks, xs, jobs = [], [], []
    out = torch.full((len(Ms), 4, N + pad), 7.0, dtype=torch.float32, device=dev)
    for i, M in enumerate(Ms):
        blk = gguf.quantize(synth.normal(40 + i, 2, (N + 7 * i) * K, 0.02), 12)
        blks.append(blk)
        xs.append(_torch_x(synth.normal(40 + i, 1, M * K).reshape(M, K), xtype, dev))
        w = ops.Tensor.quantized(torch.from_numpy(blk).to(dev), 12, N + 7 * i, K)
        jobs.append(ops.MatmulJob(w, ops.Tensor.from_torch(xs[i]), out[i, :M, :N], M, 7 * i))
    ops.dispatch_batch_matmul_multi(g, jobs, N, K)
    torch.cuda.synchronize()
    for i, M in enumerate(Ms):
        single, xr = _run(dev, blks[i], 12, _x_as_f32(xs[i]), xtype, N, 7 * i)
        got = out[i, :M, :N].cpu().numpy()
        assert np.array_equal(got, single), i
        ref = orc.batch_matmul(blks[i], 12, xr, N, K, M, 7 * i)
        assert rel_l2(got, ref) <= 1e-5, (i, rel_l2(got, ref))
        assert (out[i, M:] == 7.0).all() and (out[i, :, N:] == 7.0).all(), i


@pytest.mark.parametrize("Ms,split,f,K,xtype,o2", [
    ((4608,), 768, 1024, 512, 30, 30),     # one job on the two-pass kernel: Q|K|V part + SwiGLU part
    ((512, 3584), 0, 1024, 512, 30, 1),    # two jobs (text + image stream), SwiGLU only, f16 output2
    ((1000,), 256, 512, 512, 30, 30),      # fewer tokens: the GEMM into the workspace, then the glue
    ((2304,), 512, 760, 768, 0, 30),       # f32 activations (bf16 operands against Q4_K): the glue path
])
def test_multi_split_swiglu(orc, dev, Ms, split, f, K, xtype, o2):
    """LLMR_EPI_SPLIT_SWIGLU, the reference's Flux.2 linear1 and MLP
    in-projection (flux_dit.c3:917-931, 1013-1018, 1049-1055): weight rows
    [split, split + f) are a SwiGLU gate, the next f its up; features below
    split are stored in f32, silu(gate) * up of every output into a 16-bit
    buffer. Against the oracle's GEMM of all rows, then silu and the product
    in f32, on sampled rows of every job."""
    import torch
    from llmr_amd import capi, gguf, ops, synth
    N = split + 2 * f
    g = ops.default_graph()
    odt = torch.bfloat16 if o2 == 30 else torch.float16
    blks, xs, jobs, ys, y2s = [], [], [], [], []
    for i, M in enumerate(Ms):
        blk = gguf.quantize(synth.normal(80 + i, 2, N * K, 0.02), gguf.GGML_Q4_K)
        x = _torch_x(synth.normal(90 + i, 1, M * K).reshape(M, K), xtype, dev)
        y = torch.full((M, max(split, 4)), 7.0, device=dev)
        y2 = torch.zeros((M, f), dtype=odt, device=dev)
        blks.append(blk)
        xs.append(x)
        ys.append(y)
        y2s.append(y2)
        w = ops.Tensor.quantized(torch.from_numpy(blk).to(dev), 12, N, K)
        jobs.append(ops.MatmulJob(w, ops.Tensor.from_torch(x), y[:, :split] if split else None, M, 0,
                                  None, y2))
    print(f"split swiglu: jobs {Ms} split {split} f {f} K {K} x {xtype} output2 {o2}", flush=True)
    ops.dispatch_batch_matmul_multi(g, jobs, N, K, capi.EPI_SPLIT_SWIGLU, split)
    torch.cuda.synchronize()
    for i, M in enumerate(Ms):
        rows = _sample_rows(M)
        ref = orc.batch_matmul(blks[i], 12, _x_as_f32(xs[i]), N, K, M, 0, rows=rows.astype(np.uint32))
        ref2 = orc.silu(ref[:, split:split + f]) * ref[:, split + f:]
        got2 = y2s[i].float().cpu().numpy()[rows]
        err2 = rel_l2(got2, ref2)
        print(f"  job {i}: silu(gate) * up rel L2 {err2:.2e}", end="")
        assert np.all(np.isfinite(got2)) and err2 <= TOL
        if split:
            err = rel_l2(ys[i].cpu().numpy()[rows, :split], ref[:, :split])
            print(f", plain part rel L2 {err:.2e}", end="")
            assert err <= TOL
        print()


@pytest.mark.parametrize("N,xtype", [(18432, 30), (9216, 0)])
def test_multi_gemv_group_flux_modulation(orc, dev, N, xtype):
    """The Flux.1-dev modulation projections of one step at full size: 38
    one-token jobs of K = 3072 (19 double blocks x image/text at N = 18432,
    or 38 single blocks at N = 9216) in one grouped launch, stored with a
    row stride past N. Three weights are shared round-robin so the host
    quantizes only three; sampled jobs equal their single-job launch bit for
    bit, job 0 the oracle."""
    import torch
    from llmr_amd import gguf, ops, synth
    K, J = 3072, 38
    g = ops.default_graph()
    blks = [gguf.quantize(synth.normal(60 + i, 2, N * K, 0.02), 12) for i in range(3)]
    wts = [ops.Tensor.quantized(torch.from_numpy(b).to(dev), 12, N, K) for b in blks]
    xs = [_torch_x(synth.normal(70 + j, 1, K).reshape(1, K), xtype, dev) for j in range(J)]
    out = torch.full((J, 1, N + 64), 7.0, dtype=torch.float32, device=dev)
    jobs = [ops.MatmulJob(wts[j % 3], ops.Tensor.from_torch(xs[j]), out[j, :, :N], 1, 0) for j in range(J)]
    ops.dispatch_batch_matmul_multi(g, jobs, N, K)
    torch.cuda.synchronize()
    assert (out[:, :, N:] == 7.0).all()
    for j in (0, 1, 2, 17, 36, 37):
        single, xr = _run(dev, blks[j % 3], 12, _x_as_f32(xs[j]), xtype, N, 0)
        got = out[j, :, :N].cpu().numpy()
        assert np.array_equal(got, single), j
        if j == 0:
            ref = orc.batch_matmul(blks[0], 12, xr, N, K, 1, 0)
            assert rel_l2(got, ref) <= 1e-5, rel_l2(got, ref)


@pytest.mark.parametrize("M,xtype", [(4096, 30), (300, 30), (700, 0)])
def test_multi_split_gelu(orc, dev, M, xtype):
    """Features [0, split) to a strided f32 output, the rest gelu'd into a
    bf16 column slice: the persistent epilogue (4096 tokens) and the
    workspace path (few tiles; f32 input)."""
    import torch
    from llmr_amd import capi, ops
    N, K, split = 2304, 512, 1000
    blks, xs, wts = _multi_setup(dev, 12, (M,), N, K, xtype, 32)
    q = torch.zeros(M, split + 24, dtype=torch.float32, device=dev)
    cat = torch.zeros(M, 64 + N - split, dtype=torch.bfloat16, device=dev)
    job = ops.MatmulJob(wts[0], ops.Tensor.from_torch(xs[0]), q[:, :split], M, 0, None, cat[:, 64:])
    ops.dispatch_batch_matmul_multi(ops.default_graph(), [job], N, K, capi.EPI_SPLIT_GELU, split=split)
    torch.cuda.synchronize()
    rows = _sample_rows(M)
    ref = orc.batch_matmul(blks[0], 12, _x_as_f32(xs[0]), N, K, M, 0, rows=rows)
    ri = torch.from_numpy(rows).to(dev)
    assert rel_l2(q[ri, :split].cpu().numpy(), ref[:, :split]) <= TOL
    gel = orc.gelu(ref[:, split:])
    assert rel_l2(cat[ri, 64:].float().cpu().numpy(), gel) <= TOL
    assert (q[:, split:] == 0).all() and (cat[:, :64].float() == 0).all()


def test_multi_fused_equals_unfused_at_flux_shapes(dev):
    """Full Flux double-block shapes (512 text + 4096 image tokens, dim 3072):
    the grouped launch with gated-residual and gelu epilogues equals plain
    GEMM calls followed by the glue kernels (the same products; the fused gelu
    differs from the glue's in the last f32 bits, so the bf16 outputs agree to
    one bf16 ulp)."""
    import torch
    from llmr_amd import capi, glue, ops
    d, m, nt, ni = 3072, 12288, 512, 4096
    S = nt + ni
    g = ops.default_graph()
    wq = [glue.synth_q4k(m, d, 900 + i, device=dev) for i in range(2)]
    wd = [glue.synth_q4k(d, m, 910 + i, device=dev) for i in range(2)]
    x = torch.randn(S, d, device=dev).to(torch.bfloat16)
    gates = [torch.randn(d, device=dev) for _ in range(2)]
    sl = (slice(0, nt), slice(nt, S))
    fa = torch.empty(S, m, dtype=torch.bfloat16, device=dev)
    dummy = torch.empty(S, 16, device=dev)
    jobs = [ops.MatmulJob(ops.Tensor.quantized(wq[i], 12, m, d), ops.Tensor.from_torch(x[sl[i]]), dummy[sl[i]],
                          S - nt if i else nt, 0, None, fa[sl[i]]) for i in range(2)]
    ops.dispatch_batch_matmul_multi(g, jobs, m, d, capi.EPI_SPLIT_GELU, split=0)
    h = torch.randn(S, d, device=dev)
    h_ref = h.clone()
    jobs = [ops.MatmulJob(ops.Tensor.quantized(wd[i], 12, d, m), ops.Tensor.from_torch(fa[sl[i]]), h[sl[i]],
                          S - nt if i else nt, 0, gates[i]) for i in range(2)]
    ops.dispatch_batch_matmul_multi(g, jobs, d, m, capi.EPI_GATED_RESIDUAL)
    # unfused: plain GEMMs + glue
    for i in range(2):
        f = ops.batch_matmul(wq[i], 12, x[sl[i]].contiguous(), m)
        fa_u = torch.empty_like(fa[sl[i]])
        glue.activation(f, fa_u, capi.ACT_GELU_TANH)
        diff = (fa_u.float() - fa[sl[i]].float()).abs()
        assert (diff <= 2.0 ** -7 * fa_u.float().abs() + 1e-6).all(), float(diff.max())
        t = ops.batch_matmul(wd[i], 12, fa[sl[i]].contiguous(), d)
        glue.gated_residual(h_ref[sl[i]], t, gates[i], capi.GATE_LINEAR)
    torch.cuda.synchronize()
    err = float((h - h_ref).abs().max() / h_ref.abs().max())
    assert err < 1e-5, err


@pytest.mark.parametrize("wtype,xtype", [(8, 1), (8, 30), (12, 1), (12, 30), (12, 0)])
def test_two_pass_bit_identical_to_one_pass(dev, wtype, xtype):
    """From 2048 tokens the weight is dequantized once into a 16-bit image and
    multiplied by the all-DMA kernel; fewer tokens run the one-pass kernels.
    Both multiply the same operands in the same MFMA order, so rows of a
    4100-token launch (two-pass) equal the same rows of a 1000-token launch
    (one-pass) bit for bit: ragged N, row_offset into a fused weight."""
    import torch
    from llmr_amd import ops
    M, N, K, ro = 4100, 4100, 768, 16
    w = _weights(dev, wtype, N + ro, K, 90 + wtype)
    g = torch.Generator(device="cpu").manual_seed(wtype * 100 + xtype)
    x = torch.randn(M, K, generator=g)
    x = (x if xtype == 0 else x.to(torch.float16 if xtype == 1 else torch.bfloat16)).to(dev)
    y = ops.batch_matmul(w, wtype, x, N, row_offset=ro)
    part = ops.batch_matmul(w, wtype, x[1000:2000].contiguous(), N, row_offset=ro)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all())
    assert torch.equal(y[1000:2000], part)


@pytest.mark.parametrize("xtype", [1, 30, 0])
def test_swiglu_two_pass_bit_identical_to_one_pass(dev, xtype):
    """The SwiGLU from 2048 tokens (gate and up dequantized into one 16-bit
    image in the fused kernel's row arrangement) equals the one-pass fused
    SwiGLU on the same rows bit for bit."""
    import torch
    from llmr_amd import gguf, ops, synth
    M, N, K = 2300, 1036, 640
    wg = torch.from_numpy(gguf.quantize(synth.normal(95, 1, N * K, 0.02), 8)).to(dev)
    wu = torch.from_numpy(gguf.quantize(synth.normal(95, 2, N * K, 0.02), 8)).to(dev)
    g = torch.Generator(device="cpu").manual_seed(96 + xtype)
    x = torch.randn(M, K, generator=g)
    x = (x if xtype == 0 else x.to(torch.float16 if xtype == 1 else torch.bfloat16)).to(dev)
    y = ops.batch_matmul_swiglu(wg, wu, x, N)
    part = ops.batch_matmul_swiglu(wg, wu, x[700:1900].contiguous(), N)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all())
    assert torch.equal(y[700:1900], part)


def test_multi_two_pass_jobs_equal_single_launches(dev):
    """A grouped pair of 300 + 2000 tokens (two-pass with one image per job)
    equals each job's own single launch, for a strided store: bit for bit
    for the 2000 tokens (the one-pass persistent kernel, same MFMA order),
    to f32 summation order for the 300 (a split-K launch on its own)."""
    import torch
    from llmr_amd import ops
    Ms, N, K = (300, 2000), 4096, 512
    blks, xs, wts = _multi_setup(dev, 12, Ms, N, K, 30, 41)
    out = torch.zeros(sum(Ms), N + 32, dtype=torch.float32, device=dev)
    views = (out[:Ms[0], :N], out[Ms[0]:, :N])
    jobs = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), views[i], Ms[i], 8 * i) for i in range(2)]
    ops.dispatch_batch_matmul_multi(ops.default_graph(), jobs, N, K)
    torch.cuda.synchronize()
    for i in range(2):
        single = ops.batch_matmul(torch.from_numpy(blks[i]).to(dev), 12, xs[i], N, row_offset=8 * i)
        torch.cuda.synchronize()
        if i == 1:
            assert torch.equal(views[i], single), i
        else:
            assert rel_l2(views[i].cpu().numpy(), single.cpu().numpy()) < 1e-6, i
    assert (out[:, N:] == 0).all()


@pytest.mark.parametrize("wtype,xtype", [(12, 30), (8, 1)])
def test_multi_prebuilt_images_bit_identical(dev, wtype, xtype):
    """llmr_batch_matmul_multi_images with weight images built ahead by
    llmr_build_weight_image (on a second stream, ordered by an event) gives
    the bits of llmr_batch_matmul_multi for a grouped two-pass pair (300 +
    2000 tokens, row offsets 0 and 8) with each epilogue (strided store, gated
    residual, split gelu); a pair too small for the persistent kernels
    ignores its images."""
    import torch
    from llmr_amd import capi, ops
    g = ops.default_graph()
    Ms, N, K = (300, 2000), 4096, 512
    blks, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 43)
    n = ops.weight_image_bytes(N, K)
    imgs = [torch.full((n,), 0xAB, dtype=torch.uint8, device=dev) for _ in range(2)]
    side = torch.cuda.Stream()
    built = torch.cuda.Event()
    with torch.cuda.stream(side):
        for i in range(2):
            ops.build_weight_image(g, wts[i], N, K, 8 * i, xtype, imgs[i])
        built.record(side)
    torch.cuda.current_stream().wait_event(built)
    g.bind_stream()
    gate = torch.randn(N, device=dev)
    h0 = torch.randn(sum(Ms), N + 32, device=dev)
    for epi, split in ((capi.EPI_STORE, 0), (capi.EPI_GATED_RESIDUAL, 0), (capi.EPI_SPLIT_GELU, 1536)):
        outs = []
        for use in (False, True):
            out = h0.clone()
            o2 = torch.full((sum(Ms), N - split + 16), 3.0, dtype=torch.bfloat16, device=dev)
            jobs = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]),
                                  (out[:Ms[0], :N], out[Ms[0]:, :N])[i], Ms[i], 8 * i,
                                  gate if epi == capi.EPI_GATED_RESIDUAL else None,
                                  (o2[:Ms[0], :N - split], o2[Ms[0]:, :N - split])[i]
                                  if epi == capi.EPI_SPLIT_GELU else None) for i in range(2)]
            ops.dispatch_batch_matmul_multi(g, jobs, N, K, epi, split, images=imgs if use else None)
            torch.cuda.synchronize()
            outs.append((out, o2))
        assert torch.equal(outs[0][0], outs[1][0]), epi
        assert torch.equal(outs[0][1], outs[1][1]), epi
        assert not torch.equal(outs[1][0], h0), epi
    # a pair with too few tiles for the persistent kernels runs its own path
    small = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i][:40]), torch.empty(40, 256, device=dev), 40, 8 * i)
             for i in range(2)]
    ref = [torch.empty(40, 256, device=dev) for _ in range(2)]
    ops.dispatch_batch_matmul_multi(g, small, 256, K, images=imgs)
    ops.dispatch_batch_matmul_multi(g, [ops.MatmulJob(j.weight, j.input, r, 40, j.row_offset)
                                        for j, r in zip(small, ref)], 256, K)
    torch.cuda.synchronize()
    for j, r in zip(small, ref):
        assert torch.equal(j.output, r)


@pytest.mark.parametrize("wtype,xtype,Ms,N,K,N2,K2", [
    (12, 30, (512, 3584), 3072, 512, 2304, 3072),   # 192 tiles: 64 tile-less workgroups
    (12, 30, (300, 2000), 4096, 512, 1024, 4096),   # 160 tiles, next K = 4096
    (8, 1, (4608,), 3328, 512, 640, 1536),          # 234 tiles, ragged next N (640), Q8_0
    (12, 30, (4608,), 4096, 256, 256, 256),          # 288 tiles: a second round of 32
    (12, 30, (2048,), 7936, 256, 1024, 3072),       # 248 tiles: 16 of 48 items fused, 32 after
])
def test_multi_next_images_built_by_idle_workgroups(dev, wtype, xtype, Ms, N, K, N2, K2):
    """A call's next_images (part built by its two-pass GEMM's workgroups
    without a tile in the last round, the rest right after) equal the images
    llmr_build_weight_image builds, byte for byte, and the call's own output
    is the plain call's; the next group's call on them gives the plain bits."""
    import torch
    from llmr_amd import capi, gguf, ops, synth
    g = ops.default_graph()
    blks, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 47)
    nw = [ops.Tensor.quantized(torch.from_numpy(gguf.quantize(synth.normal(47, 60 + i, (N2 + 16) * K2, 0.02),
                                                              wtype)).to(dev), wtype, N2 + 16, K2)
          for i in range(len(Ms))]
    nb = ops.weight_image_bytes(N2, K2)
    chained = [torch.zeros(nb, dtype=torch.uint8, device=dev) for _ in Ms]
    direct = [torch.zeros(nb, dtype=torch.uint8, device=dev) for _ in Ms]
    out_a = torch.zeros(sum(Ms), N, device=dev)
    out_b = torch.zeros(sum(Ms), N, device=dev)
    rows = [sum(Ms[:i]) for i in range(len(Ms) + 1)]

    def jobs(out):
        return [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), out[rows[i]:rows[i + 1]], Ms[i], 8 * i)
                for i in range(len(Ms))]
    nxt = ops.NextImages.group(nw, N2, K2, chained, row_offsets=tuple(16 * i for i in range(len(Ms))))
    ops.dispatch_batch_matmul_multi(g, jobs(out_a), N, K, next_images=nxt)
    ops.dispatch_batch_matmul_multi(g, jobs(out_b), N, K)
    for i in range(len(Ms)):
        ops.build_weight_image(g, nw[i], N2, K2, 16 * i, xtype, direct[i])
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    for i in range(len(Ms)):
        assert torch.equal(chained[i], direct[i]), i
    # the next group on the chained images
    x2 = [_torch_x(synth.normal(47, 70 + i, Ms[i] * K2).reshape(Ms[i], K2), xtype, dev) for i in range(len(Ms))]
    y_a = torch.zeros(sum(Ms), N2, device=dev)
    y_b = torch.zeros(sum(Ms), N2, device=dev)
    j2 = lambda y: [ops.MatmulJob(nw[i], ops.Tensor.from_torch(x2[i]), y[rows[i]:rows[i + 1]], Ms[i], 16 * i)  # noqa: E731
                    for i in range(len(Ms))]
    ops.dispatch_batch_matmul_multi(g, j2(y_a), N2, K2, images=chained)
    ops.dispatch_batch_matmul_multi(g, j2(y_b), N2, K2)
    torch.cuda.synchronize()
    assert torch.equal(y_a, y_b)


@pytest.mark.parametrize("wtype,M,N,K,xtype", [(8, 256, 3072, 3072, 0), (12, 300, 520, 1024, 30), (8, 96, 4096, 4096, 1),
                                               (8, 64, 1024, 4096, 0), (12, 320, 640, 3072, 0)])
def test_split_k_matches_oracle_and_repeats(orc, dev, wtype, M, N, K, xtype):
    """Launches with few tiles split K over several workgroup rows (or, on the
    few-token kernel, over the waves of a workgroup) and sum the partials in
    split order: within the GEMM bar of the oracle, and the same bits on every
    call. 320 x 640 x 3072 once planned an eleventh split with no K stage."""
    import torch
    from llmr_amd import gguf, synth
    blk = gguf.quantize(synth.normal(97, 2, N * K, 0.02), wtype)
    x = synth.normal(97, 1, M * K).reshape(M, K)
    y, xr = _run(dev, blk, wtype, x, xtype, N)
    y2, _ = _run(dev, blk, wtype, x, xtype, N)
    ref = orc.batch_matmul(blk, wtype, xr, N, K, M, 0)
    err = rel_l2(y, ref)
    print(f"split-K wtype={wtype} M={M} N={N} K={K}: rel_l2={err:.3e}")
    assert err <= TOL
    assert np.array_equal(y, y2)


def test_weight_image_entry_points_reject_bad_arguments(dev):
    """llmr_build_weight_image / llmr_batch_matmul_multi_images /
    llmr_flash_attention_rows reject what they cannot take, with a message,
    before launching anything."""
    import ctypes
    import torch
    from llmr_amd import capi, gguf, ops, synth
    g = ops.default_graph()
    g.bind_stream()
    N, K = 512, 512
    blk = torch.from_numpy(gguf.quantize(synth.normal(5, 1, N * K, 0.02), 12)).to(dev)
    w = ops.Tensor.quantized(blk, 12, N, K)
    nb = ops.weight_image_bytes(N, K)
    img = torch.zeros(nb + 256, dtype=torch.uint8, device=dev)
    ctx = g.ctx
    with pytest.raises(capi.LlmrError, match="F16 or BF16"):
        ctx.build_weight_image(w.ptr(), 12, 0, N, K, 0, img.data_ptr(), nb)       # f32 operands
    with pytest.raises(capi.LlmrError, match="multiple of 64"):
        ctx.build_weight_image(w.ptr(), 12, 30, N, 256 + 32, 0, img.data_ptr(), nb)
    with pytest.raises(capi.LlmrError, match="256-byte aligned"):
        ctx.build_weight_image(w.ptr(), 12, 30, N, K, 0, img.data_ptr() + 16, nb)
    with pytest.raises(capi.LlmrError, match="needs"):
        ctx.build_weight_image(w.ptr(), 12, 30, N, K, 0, img.data_ptr(), nb - 1)
    x = torch.zeros(2048, K, dtype=torch.bfloat16, device=dev)
    y = torch.zeros(2048, N, device=dev)
    job = capi.MatmulJob(w.ptr(), x.data_ptr(), y.data_ptr(), None, None, 2048, 0)
    epi = capi.MatmulEpilogue(capi.EPI_STORE, N, 0, 0, 0)
    with pytest.raises(capi.LlmrError, match="256-byte aligned"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, [img.data_ptr() + 16])
    img2 = torch.zeros(nb, dtype=torch.uint8, device=dev)
    one = capi.NextWeightImage(w.ptr(), N, K, 0, 0, 0, img.data_ptr(), nb)
    nxt = capi.NextWeightImages(12, 9, (capi.NextWeightImage * 8)(*([one] * 8)))
    with pytest.raises(capi.LlmrError, match="count"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.count = 2  # images 0 and 1 in one buffer
    with pytest.raises(capi.LlmrError, match="same buffer"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.image[1] = capi.NextWeightImage(w.ptr(), N, K, 0, 0, 0, img2.data_ptr(), nb - 1)
    with pytest.raises(capi.LlmrError, match="needs"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    # a SwiGLU image of N outputs: twice the panels of the plain one
    assert ops.swiglu_weight_image_bytes(N, K) > nb
    nxt.image[1] = capi.NextWeightImage(w.ptr(), N, K, 0, 1, 0, img2.data_ptr(), nb)
    with pytest.raises(capi.LlmrError, match="needs"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.image[1] = capi.NextWeightImage(w.ptr(), N, K, 0, 2, 0, img2.data_ptr(), nb)
    with pytest.raises(capi.LlmrError, match="swiglu must be 0 or 1"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.image[1] = capi.NextWeightImage(w.ptr(), N // 2, K, 0, 0, N // 2, img2.data_ptr(), nb)
    with pytest.raises(capi.LlmrError, match="up_offset needs swiglu"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.image[1] = capi.NextWeightImage(w.ptr(), N // 4, K, 0, 1, N // 8, img2.data_ptr(), nb)
    with pytest.raises(capi.LlmrError, match="up_offset below out_dim"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.image[1] = capi.NextWeightImage(w.ptr(), N, 256 + 32, 0, 0, 0, img2.data_ptr(), nb)
    with pytest.raises(capi.LlmrError, match="in_dim"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, None, nxt)
    nxt.count = 1
    with pytest.raises(capi.LlmrError, match="also an image"):
        ctx.batch_matmul_multi_images(12, 30, N, K, [job], epi, [img.data_ptr()], nxt)
    with pytest.raises(capi.LlmrError, match="F16 or BF16"):
        ctx.batch_matmul_multi_images(12, 0, N, K, [job], epi, None, nxt)
    q = torch.zeros(2, 64, 128, dtype=torch.float16, device=dev)
    o = torch.zeros(64, 264, dtype=torch.bfloat16, device=dev)
    with pytest.raises(capi.LlmrError, match="out_stride"):
        ctx.flash_attention_rows(q.data_ptr(), q.data_ptr(), q.data_ptr(), 1, o.data_ptr(), 30, 260, 128, 2, 64, 0.1)
    with pytest.raises(capi.LlmrError, match="output type"):
        ctx.flash_attention_rows(q.data_ptr(), q.data_ptr(), q.data_ptr(), 1, o.data_ptr(), 8, 264, 128, 2, 64, 0.1)
    torch.cuda.synchronize()
    assert (y == 0).all()


@pytest.mark.parametrize("wtype,xtype,Ms,N,K", [
    (12, 30, (512, 4096), 9216, 3072),   # the Flux double block's QKV: 648 tiles, room for all 73 items
    (8, 1, (4608,), 3328, 512),           # 234 tiles: room for 44 of the 73 items, the rest after the GEMM
])
def test_multi_next_images_of_two_groups(dev, wtype, xtype, Ms, N, K):
    """next_images of the two groups after this call (the Flux double block's
    QKV builds the projection's and the MLP-in's): four images of two shapes
    (N2 x K2, N3 x K3, with row offsets), numbered across all four, built
    as far as the call's idle workgroups reach and the rest after the GEMM,
    equal llmr_build_weight_image's bytes; the call's own output is the
    plain call's."""
    import torch
    from llmr_amd import gguf, ops, synth
    g = ops.default_graph()
    blks, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 53)
    # (N2, K2, row_offset): 9 + 12 + 48 + 4 items of (256-row panel, 4 K stages)
    shapes = [(640, 768, 0), (1000, 768, 8), (1536, 2048, 0), (256, 1024, 16)]
    nw = [ops.Tensor.quantized(torch.from_numpy(gguf.quantize(synth.normal(53, 60 + i, (n + ro) * k, 0.02),
                                                              wtype)).to(dev), wtype, n + ro, k)
          for i, (n, k, ro) in enumerate(shapes)]
    chained = [torch.zeros(ops.weight_image_bytes(n, k), dtype=torch.uint8, device=dev) for n, k, _ in shapes]
    direct = [torch.zeros_like(c) for c in chained]
    out_a = torch.zeros(sum(Ms), N, device=dev)
    out_b = torch.zeros(sum(Ms), N, device=dev)
    rows = [sum(Ms[:i]) for i in range(len(Ms) + 1)]

    def jobs(out):
        return [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), out[rows[i]:rows[i + 1]], Ms[i], 8 * i)
                for i in range(len(Ms))]
    nxt = ops.NextImages([ops.NextImage(w, n, k, im, ro) for w, (n, k, ro), im in zip(nw, shapes, chained)])
    ops.dispatch_batch_matmul_multi(g, jobs(out_a), N, K, next_images=nxt)
    ops.dispatch_batch_matmul_multi(g, jobs(out_b), N, K)
    for w, (n, k, ro), im in zip(nw, shapes, direct):
        ops.build_weight_image(g, w, n, k, ro, xtype, im)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    for i in range(len(shapes)):
        assert torch.equal(chained[i], direct[i]), i


@pytest.mark.parametrize("wtype,xtype,Ms,N,K", [
    (12, 30, (4608,), 3328, 512),        # 234 tiles: room for 44 of the 51 items, the SwiGLU image's last 7 after
    (8, 1, (512, 4096), 9216, 3072),     # 648 tiles: room for all of them
])
def test_multi_next_swiglu_images(dev, wtype, xtype, Ms, N, K):
    """next_images with SwiGLU-arranged entries (the Flux.2 linear1 and MLP
    in-projection): a SPLIT_SWIGLU weight's plain rows and its SwiGLU image
    in one buffer, a second weight's SwiGLU image alone (split 0, row offset)
    and a plain image, built as far as the call's idle workgroups reach and
    the rest after the GEMM, equal the same images built by a call without
    jobs byte for byte; a SPLIT_SWIGLU GEMM reading the first buffer equals
    the one that builds its own image, bit for bit."""
    import torch
    from llmr_amd import capi, gguf, ops, synth
    g = ops.default_graph()
    _, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 71)
    split, f, K1 = 512, 1000, 768          # 6 plain + 24 SwiGLU items (f % 128 != 0: a ragged panel)
    f2, K2, ro2 = 264, 1024, 16            # 12 SwiGLU items
    n3, K3, ro3 = 640, 768, 8              # 9 plain items

    def qw(seed, rows, k):
        blk = gguf.quantize(synth.normal(71, seed, rows * k, 0.02), wtype)
        return ops.Tensor.quantized(torch.from_numpy(blk).to(dev), wtype, rows, k)
    w1, w2, w3 = qw(40, split + 2 * f, K1), qw(41, ro2 + 2 * f2, K2), qw(42, ro3 + n3, K3)

    def bufs():
        return [torch.zeros(ops.split_swiglu_image_bytes(split, f, K1), dtype=torch.uint8, device=dev),
                torch.zeros(ops.swiglu_weight_image_bytes(f2, K2), dtype=torch.uint8, device=dev),
                torch.zeros(ops.weight_image_bytes(n3, K3), dtype=torch.uint8, device=dev)]

    def nxt(b):
        return (ops.NextImages.split_swiglu([w1], split, f, K1, [b[0]]) +
                ops.NextImages([ops.NextImage(w3, n3, K3, b[2], ro3)]) +
                ops.NextImages.split_swiglu([w2], 0, f2, K2, [b[1]], (ro2,)))
    chained, direct = bufs(), bufs()
    assert len(nxt(chained).entries) == 4
    out_a = torch.zeros(sum(Ms), N, device=dev)
    out_b = torch.zeros(sum(Ms), N, device=dev)
    rows = [sum(Ms[:i]) for i in range(len(Ms) + 1)]

    def jobs(out):
        return [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), out[rows[i]:rows[i + 1]], Ms[i], 8 * i)
                for i in range(len(Ms))]
    print(f"next swiglu images: w{wtype} x{xtype} jobs {Ms} {N}x{K}", flush=True)
    ops.dispatch_batch_matmul_multi(g, jobs(out_a), N, K, next_images=nxt(chained))
    ops.dispatch_batch_matmul_multi(g, jobs(out_b), N, K)
    ops.build_next_images(g, nxt(direct), xtype)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    for i in range(3):
        assert torch.equal(chained[i], direct[i]), i
    # the split-SwiGLU GEMM on the chained image and on its own
    M = 2304
    x = _torch_x(synth.normal(71, 50, M * K1).reshape(M, K1), xtype, dev)
    odt = torch.float16 if xtype == 1 else torch.bfloat16
    ys = [torch.full((M, split), 7.0, device=dev) for _ in range(2)]
    y2s = [torch.zeros((M, f), dtype=odt, device=dev) for _ in range(2)]
    for y, y2, im in ((ys[0], y2s[0], [chained[0]]), (ys[1], y2s[1], None)):
        ops.dispatch_batch_matmul_multi(g, [ops.MatmulJob(w1, ops.Tensor.from_torch(x), y, M, 0, None, y2)],
                                        split + 2 * f, K1, capi.EPI_SPLIT_SWIGLU, split, images=im)
    torch.cuda.synchronize()
    assert torch.equal(ys[0], ys[1]) and torch.equal(y2s[0], y2s[1])
    assert torch.isfinite(y2s[0].float()).all() and y2s[0].float().abs().max() > 0


@pytest.mark.parametrize("wtype,xtype", [(12, 30), (8, 1)])
def test_next_image_parts_assemble_whole_images(dev, wtype, xtype):
    """Next images that are parts of an image (whole panels: rows [256 p0,
    256 p1) of a plain image at row offset + 256 p0, outputs [128 p0, 128
    p1) of a SwiGLU image at its gate rows + 128 p0 with up_offset the
    image's output count), built by a GEMM call (as far as its idle
    workgroups reach, the rest after it), land where the whole image has
    those panels: byte for byte the whole images built by a call without
    jobs. Ragged last panels on both."""
    import torch
    from llmr_amd import gguf, ops, synth
    g = ops.default_graph()
    Ms, N, K = (4608,), 3328, 512  # 234 tiles: room for 44 items
    _, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 73)
    K2, ro = 768, 16
    f, n = 264, 640  # SwiGLU outputs (3 panels of 128), plain rows (3 panels of 256)

    def qw(seed, rows):
        blk = gguf.quantize(synth.normal(73, seed, rows * K2, 0.02), wtype)
        return ops.Tensor.quantized(torch.from_numpy(blk).to(dev), wtype, rows, K2)
    wsw, wpl = qw(40, ro + 2 * f), qw(41, ro + n)
    panel = ops.weight_image_bytes(256, K2)
    whole = [torch.zeros(ops.swiglu_weight_image_bytes(f, K2), dtype=torch.uint8, device=dev),
             torch.zeros(ops.weight_image_bytes(n, K2), dtype=torch.uint8, device=dev)]
    parts = [torch.zeros_like(t) for t in whole]
    ops.build_next_images(g, ops.NextImages([ops.NextImage(wsw, f, K2, whole[0], ro, True),
                                             ops.NextImage(wpl, n, K2, whole[1], ro)]), xtype)
    nxt = ops.NextImages([
        ops.NextImage(wsw, 128, K2, parts[0][:panel], ro, True, f),
        ops.NextImage(wpl, 256, K2, parts[1][:panel], ro),
        ops.NextImage(wsw, f - 128, K2, parts[0][panel:], ro + 128, True, f),
        ops.NextImage(wpl, n - 256, K2, parts[1][panel:], ro + 256)])
    out = torch.zeros(sum(Ms), N, device=dev)
    print(f"next image parts: w{wtype} x{xtype}", flush=True)
    ops.dispatch_batch_matmul_multi(g, [ops.MatmulJob(wts[0], ops.Tensor.from_torch(xs[0]), out, Ms[0], 0)], N, K,
                                    next_images=nxt)
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(parts[i], whole[i]), i
    assert whole[0].any() and whole[1].any()


def test_next_image_parts_random(dev):
    """Eight seeded random cases of image parts as next images of one GEMM
    call: a plain and a SwiGLU image of random ragged sizes, row offsets and
    K, each cut at a random panel into two parts listed in random order,
    equal the whole images byte for byte (both weight types)."""
    import random
    import torch
    from llmr_amd import gguf, ops, synth
    rnd = random.Random(1202)
    g = ops.default_graph()
    Ms, N, K = (4608,), 3328, 512
    for case in range(8):
        wtype = rnd.choice((8, 12))
        xtype = rnd.choice((1, 30))
        _, xs, wts = _multi_setup(dev, wtype, Ms, N, K, xtype, 90 + case)
        K2 = 256 * rnd.randint(1, 4)
        f, n = 8 * rnd.randint(17, 80), 8 * rnd.randint(33, 160)  # > one panel each
        ro_s, ro_p = 8 * rnd.randint(0, 4), 8 * rnd.randint(0, 4)

        def qw(seed, rows):
            blk = gguf.quantize(synth.normal(90 + case, seed, rows * K2, 0.02), wtype)
            return ops.Tensor.quantized(torch.from_numpy(blk).to(dev), wtype, rows, K2)
        wsw, wpl = qw(40, ro_s + 2 * f + 8), qw(41, ro_p + n + 8)
        panel = ops.weight_image_bytes(256, K2)
        whole = [torch.zeros(ops.swiglu_weight_image_bytes(f, K2), dtype=torch.uint8, device=dev),
                 torch.zeros(ops.weight_image_bytes(n, K2), dtype=torch.uint8, device=dev)]
        parts = [torch.zeros_like(t) for t in whole]
        ops.build_next_images(g, ops.NextImages([ops.NextImage(wsw, f, K2, whole[0], ro_s, True),
                                                 ops.NextImage(wpl, n, K2, whole[1], ro_p)]), xtype)
        ps = rnd.randint(1, -(-f // 128) - 1)  # the SwiGLU image's cut (panels of 128 outputs)
        pp = rnd.randint(1, -(-n // 256) - 1) if n > 256 else 1
        es = [ops.NextImage(wsw, 128 * ps, K2, parts[0][:ps * panel], ro_s, True, f),
              ops.NextImage(wsw, f - 128 * ps, K2, parts[0][ps * panel:], ro_s + 128 * ps, True, f)]
        if 256 * pp < n:
            es += [ops.NextImage(wpl, 256 * pp, K2, parts[1][:pp * panel], ro_p),
                   ops.NextImage(wpl, n - 256 * pp, K2, parts[1][pp * panel:], ro_p + 256 * pp)]
        else:
            es.append(ops.NextImage(wpl, n, K2, parts[1], ro_p))
        rnd.shuffle(es)
        out = torch.zeros(sum(Ms), N, device=dev)
        print(f"parts case {case}: w{wtype} x{xtype} K2 {K2} f {f} cut {ps} n {n} cut {pp}", flush=True)
        ops.dispatch_batch_matmul_multi(g, [ops.MatmulJob(wts[0], ops.Tensor.from_torch(xs[0]), out, Ms[0], 0)], N,
                                        K, next_images=ops.NextImages(es))
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(parts[i], whole[i]), (case, i)
