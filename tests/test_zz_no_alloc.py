"""llmr_batch_matmul_noalloc, the GEMM entry point that allocates nothing:
its scratch is the library's fixed device array. Each case calls it twice in
a row through the C-ABI, the second time with a smaller input, and compares
every output with llmr_batch_matmul's on the same inputs: bit for bit where
both run the same kernels or the no-allocation call runs the one-pass
kernels in place of the two-pass path (the same bits), to f32 summation
order where it runs fewer K splits. A fresh context's no-allocation calls
leave the device's free memory unchanged, and calls of one context on two
streams are ordered around the shared scratch."""
import pytest
import torch

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 0, 1, 30


def _weights(dev, wtype, rows, K, seed):
    from llmr_amd import glue, gguf, synth
    if wtype == 12:
        return glue.synth_q4k(rows, K, seed, device=dev)
    return torch.from_numpy(gguf.quantize(synth.normal(seed, 2, rows * K, 0.02), wtype)).to(dev)


def _x(dev, M, K, xtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    return (x if xtype == F32 else x.to(torch.float16 if xtype == F16 else torch.bfloat16)).to(dev)


def _both(dev, w, wtype, x, xtype, N, row_offset=0):
    from llmr_amd import ops
    g = ops.default_graph()
    g.bind_stream()
    M, K = x.shape
    y_ref = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    y = torch.full((M, N), -7.0, dtype=torch.float32, device=dev)
    g.ctx.batch_matmul(w.data_ptr(), wtype, x.data_ptr(), xtype, y_ref.data_ptr(), N, K, M, row_offset)
    g.ctx.batch_matmul_noalloc(w.data_ptr(), wtype, x.data_ptr(), xtype, y.data_ptr(), N, K, M, row_offset)
    torch.cuda.synchronize()
    return y, y_ref


# (wtype, xtype, N, K, (M first call, M second call), row_offset, what the
# scratch holds). Where llmr_batch_matmul's plan fits the array both calls run
# the same kernels (same bits); a launch whose weight image does not fit runs
# the one-pass kernels (same bits as the two-pass path); one whose split-K
# partials do not fit runs fewer splits (the same sums in another order:
# compared to f32 rounding, far inside the GEMM bar of relative L2 1e-2).
CASES = [
    (8, F32, 3072, 3072, (256, 64), 0, "nothing (the single Q8_0 linear), then split-K partials"),
    (12, F32, 4096, 1024, (4096, 2304), 8, "f32 activations as bf16 + the weight image"),
    (12, BF16, 12288, 3072, (2560, 2304), 0, "nothing: one-pass in place of a 75 MB weight image"),
    (12, BF16, 3072, 3072, (4608, 2048), 0, "the weight image; then fewer splits than llmr_batch_matmul"),
    (8, F16, 1000, 2048, (300, 40), 4, "split-K partials, ragged N"),
]


@pytest.mark.parametrize("wtype,xtype,N,K,Ms,row_offset,what", CASES)
def test_noalloc_matches_batch_matmul_twice(dev, wtype, xtype, N, K, Ms, row_offset, what):
    from conftest import rel_l2
    w = _weights(dev, wtype, N + row_offset, K, 60 + wtype)
    for i, M in enumerate(Ms):
        x = _x(dev, M, K, xtype, 1000 * i + M)
        print(f"noalloc wtype={wtype} xtype={xtype} M={M} N={N} K={K} ({what})", flush=True)
        y, y_ref = _both(dev, w, wtype, x, xtype, N, row_offset)
        assert bool(torch.isfinite(y_ref).all())
        assert bool(torch.isfinite(y).all())
        err = rel_l2(y.cpu().numpy(), y_ref.cpu().numpy())
        exact = torch.equal(y, y_ref)
        print(f"  rel L2 {err:.2e}, identical {exact}")
        assert err <= 1e-5, (M, err)
        if not (wtype == 12 and xtype == BF16 and N == 3072 and M == 2048):
            assert exact, M


def test_noalloc_f32_beyond_scratch_runs_tiled(dev):
    """f32 activations of 4608 x 4096 would need a 36 MiB 16-bit copy for the
    persistent kernels, more than the 32 MiB array: the call runs the tiled
    kernel, which rounds them in registers to the same operands, so it agrees
    with llmr_batch_matmul to f32 summation order."""
    from conftest import rel_l2
    N, K, M = 4096, 4096, 4608
    w = _weights(dev, 12, N, K, 77)
    x = _x(dev, M, K, F32, 5)
    print("noalloc f32 4608 x 4096 x 4096 Q4_K (tiled in place of the persistent kernels)", flush=True)
    y, y_ref = _both(dev, w, 12, x, F32, N)
    assert bool(torch.isfinite(y).all())
    err = rel_l2(y.cpu().numpy(), y_ref.cpu().numpy())
    print(f"  rel L2 {err:.2e}")
    assert err <= 1e-5


def test_noalloc_allocates_nothing_on_a_fresh_context(dev):
    """A context that has never run a GEMM calls only llmr_batch_matmul_noalloc,
    on launches whose plans use scratch (split-K partials, a 16-bit copy of f32
    activations, a weight image): the device's free memory is the same before
    and after. (The kernels' code is loaded first through another context.)"""
    from llmr_amd import capi, ops
    cases = [(8, F32, 3072, 3072, 64), (12, F32, 4096, 1024, 2304), (12, BF16, 3072, 3072, 4608)]
    data = []
    for wtype, xtype, N, K, M in cases:
        w = _weights(dev, wtype, N, K, 90 + wtype)
        x = _x(dev, M, K, xtype, 3 + M)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        data.append((w, wtype, x, xtype, y, N, K, M))
    warm = ops.default_graph()
    warm.bind_stream()
    for w, wtype, x, xtype, y, N, K, M in data:  # load every kernel's code
        warm.ctx.batch_matmul_noalloc(w.data_ptr(), wtype, x.data_ptr(), xtype, y.data_ptr(), N, K, M, 0)
    torch.cuda.synchronize()
    ctx = capi.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    free0 = torch.cuda.mem_get_info()[0]
    for w, wtype, x, xtype, y, N, K, M in data:
        print(f"fresh context noalloc wtype={wtype} xtype={xtype} M={M} N={N} K={K}", flush=True)
        ctx.batch_matmul_noalloc(w.data_ptr(), wtype, x.data_ptr(), xtype, y.data_ptr(), N, K, M, 0)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    ctx.close()
    assert free1 == free0, (free0, free1)
    assert all(bool(torch.isfinite(d[4]).all()) for d in data)


def test_noalloc_two_streams_of_one_context(dev):
    """Two no-allocation calls whose plans use the scratch (split-K partials),
    issued on two streams of one context one after the other: the second
    waits for the first stream's work up to the switch, so both results are
    llmr_batch_matmul's."""
    from llmr_amd import capi
    N, K = 3072, 3072
    w = _weights(dev, 8, N, K, 31)
    xs = [_x(dev, 64, K, F32, 11), _x(dev, 64, K, F32, 12)]
    ys = [torch.full((64, N), -1.0, device=dev) for _ in xs]
    refs = [torch.empty((64, N), device=dev) for _ in xs]
    ctx = capi.Context(0)
    s0, s1 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    print("noalloc on two streams of one context: 64 x 3072 x 3072 Q8_0 f32 (split-K partials)", flush=True)
    for st, x, y in ((s0, xs[0], ys[0]), (s1, xs[1], ys[1])):
        ctx.set_stream(st.cuda_stream)
        ctx.batch_matmul_noalloc(w.data_ptr(), 8, x.data_ptr(), F32, y.data_ptr(), N, K, 64, 0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for x, r in zip(xs, refs):
        ctx.batch_matmul(w.data_ptr(), 8, x.data_ptr(), F32, r.data_ptr(), N, K, 64, 0)
    torch.cuda.synchronize()
    ctx.close()
    for y, r in zip(ys, refs):
        assert torch.equal(y, r)
