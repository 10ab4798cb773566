"""llmr_batch_matmul_noalloc, the GEMM entry point that allocates nothing:
its scratch is the library's fixed device array. Each case calls it twice in
a row through the C-ABI, the second time with a smaller input, and compares
every output with llmr_batch_matmul's on the same inputs: bit for bit where
both run the same kernels or the no-allocation call runs the one-pass
kernels in place of the two-pass path (the same bits), to f32 summation
order where it runs fewer K splits. A call whose scratch would not fit is
refused before anything is launched."""
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
    (8, F32, 3072, 3072, (256, 64), 0, "split-K partials (the single Q8_0 linear)"),
    (12, F32, 4096, 1024, (4096, 2304), 8, "f32 activations as fp16 + the weight image"),
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


def test_noalloc_refuses_scratch_beyond_its_array(dev):
    """f32 activations of 4608 x 4096 on a persistent-kernel launch need 36 MiB
    of fp16 copy, more than the 32 MiB array: refused with a message, output
    untouched."""
    from llmr_amd import capi, ops
    N, K, M = 4096, 4096, 4608
    w = _weights(dev, 12, N, K, 77)
    x = _x(dev, M, K, F32, 5)
    y = torch.full((M, N), 3.0, dtype=torch.float32, device=dev)
    g = ops.default_graph()
    g.bind_stream()
    rc = capi.lib().llmr_batch_matmul_noalloc(g.ctx._h, w.data_ptr(), 12, x.data_ptr(), F32, y.data_ptr(), N, K, M,
                                              0)
    torch.cuda.synchronize()
    assert rc == capi.LLMR_ERR_INVALID_ARG
    assert "scratch" in capi.last_error()
    assert bool((y == 3.0).all())
    # the same product with bf16 activations needs no scratch
    xb = x.to(torch.bfloat16)
    yb, yb_ref = _both(dev, w, 12, xb, BF16, N)
    assert torch.equal(yb, yb_ref)
