"""llmr_batch_matmul_multi_qkv: a QKV projection with the head norm, RoPE
and head-major Q/K/V done on its result in the GEMM epilogue
(flux_dit.c3:786-863, 1005-1040; dit.c3:1434-1473), against the unfused
composition: llmr_batch_matmul_multi, then llmr_qkv_heads on its f32
result (each of which the oracle checks: test_gpu_gemm.py, test_gpu_glue.py).
Bit for bit on both paths the call takes: the two-pass persistent kernel's
epilogue (from a few thousand tokens), and the GEMM into the workspace plus
the glue pass. The
cases cover pairs of jobs with their own norms and first rows; the STORE,
SPLIT_GELU and SPLIT_SWIGLU epilogues; an odd head count, where a tile
straddles the Q | K | V end; and f16 and bf16 Q/K/V."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

STORE, GELU, SWIGLU = 0, 2, 3


def _x(seed, M, K, xtype, dev):
    import torch
    from llmr_amd import synth
    t = torch.from_numpy(synth.normal(seed, 1, M * K).reshape(M, K))
    return t.to({0: torch.float32, 1: torch.float16, 30: torch.bfloat16}[xtype]).to(dev)


def _weight(seed, wtype, N, K, dev):
    import torch
    from llmr_amd import gguf, ops, synth
    blk = gguf.quantize(synth.normal(seed, 2, N * K, 0.02), wtype)
    return ops.Tensor.quantized(torch.from_numpy(blk).to(dev), wtype, N, K)


# wtype, xtype, job tokens, heads, K, epilogue, MLP columns past Q | K | V,
# RoPE, norms ("qk", "q", ""), Q/K/V dtype, prebuilt weight images; the path
@pytest.mark.parametrize("wtype,xtype,Ms,H,K,epi,extra,rope,norms,odt,images", [
    (12, 30, (512, 3584), 8, 512, STORE, 0, True, "qk", "f16", False),      # two-pass, a pair
    (12, 30, (512, 3584), 8, 512, STORE, 0, True, "qk", "f16", True),       # the same from weight images
    (12, 30, (4096,), 4, 512, GELU, 1024, True, "qk", "f16", False),        # two-pass, linear1 with gelu
    (12, 30, (4096,), 4, 512, SWIGLU, 512, True, "qk", "bf16", False),      # two-pass, linear1 with SwiGLU
    (8, 30, (4096,), 6, 768, STORE, 0, True, "qk", "f16", False),           # two-pass Q8_0 (Z-Image QKV)
    (12, 1, (1536,), 16, 256, STORE, 0, True, "qk", "bf16", False),         # one-pass sizes: GEMM + glue
    (8, 30, (1536,), 16, 256, STORE, 0, True, "qk", "f16", False),          # the same for Q8_0
    (12, 30, (5120,), 3, 256, GELU, 512, False, "q", "f16", False),         # odd H: a straddling tile
    (12, 30, (100, 37), 2, 512, STORE, 0, True, "qk", "f16", False),        # few tokens: GEMM + glue
    (12, 0, (2048,), 4, 512, STORE, 0, True, "", "f16", False),             # f32 activations: GEMM + glue
])
def test_qkv_epilogue_bit_identical_to_gemm_then_qkv_heads(dev, wtype, xtype, Ms, H, K, epi, extra, rope, norms,
                                                          odt, images):
    import torch
    from llmr_amd import capi, glue, ops
    g = ops.default_graph()
    qkv = 3 * H * 128
    split = qkv if epi != STORE else 0
    N = qkv + (2 * extra if epi == SWIGLU else extra)
    n2 = extra
    S = sum(Ms) + 16  # rows past the jobs' stay untouched
    odtype = torch.float16 if odt == "f16" else torch.bfloat16
    print(f"qkv epilogue: w {wtype} x {xtype} jobs {Ms} H {H} K {K} epi {epi} extra {extra} rope {rope} "
          f"norms {norms!r} {odt} images {images}", flush=True)
    wts = [_weight(300 + i, wtype, N, K, dev) for i in range(len(Ms))]
    xs = [_x(310 + i, M, K, xtype, dev) for i, M in enumerate(Ms)]
    gen = torch.Generator().manual_seed(5)
    cos_t = torch.randn(S, 64, generator=gen).to(dev)
    sin_t = torch.randn(S, 64, generator=gen).to(dev)
    qn = [(1 + 0.1 * torch.randn(128, generator=gen)).to(dev) for _ in Ms]
    kn = [(1 + 0.1 * torch.randn(128, generator=gen)).to(dev) for _ in Ms]
    row0 = np.concatenate([[0], np.cumsum(Ms)[:-1]]).tolist()
    hjobs = [(qn[i] if "q" in norms else None, kn[i] if "k" in norms else None, row0[i]) for i in range(len(Ms))]
    tables = (cos_t, sin_t) if rope else None
    imgs = None
    if images:
        nb = ops.weight_image_bytes(N, K)
        imgs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in Ms]
        for w, im in zip(wts, imgs):
            ops.build_weight_image(g, w, N, K, 0, xtype, im)

    def outs():
        fill = torch.full((H, S, 128), float("nan"), dtype=odtype, device=dev)
        return fill, fill.clone(), fill.clone(), torch.full((sum(Ms), max(n2, 4)), 3.0, dtype=torch.bfloat16,
                                                            device=dev)

    # the unfused composition: f32 result, then qkv_heads per job
    q0, k0, v0, o20 = outs()
    y = torch.full((sum(Ms), N), 7.0, device=dev)
    r = np.concatenate([[0], np.cumsum(Ms)]).tolist()
    jobs = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), y[r[i]:r[i + 1], :split or N], M, 0, None,
                          o20[r[i]:r[i + 1], :n2] if extra else None) for i, M in enumerate(Ms)]
    ops.dispatch_batch_matmul_multi(g, jobs, N, K, epi, split)
    for i, M in enumerate(Ms):
        glue.qkv_heads(y[r[i]:r[i + 1]], H, q0, k0, v0, row0[i], hjobs[i][0], hjobs[i][1], 1e-6, tables, g=g)
    # the fused call
    q1, k1, v1, o21 = outs()
    jobs = [ops.MatmulJob(wts[i], ops.Tensor.from_torch(xs[i]), None, M, 0, None,
                          o21[r[i]:r[i + 1], :n2] if extra else None) for i, M in enumerate(Ms)]
    ops.dispatch_batch_matmul_multi(g, jobs, N, K, epi, split, images=imgs,
                                    heads=ops.QkvHeads(q1, k1, v1, H, hjobs, 1e-6, tables))
    torch.cuda.synchronize()
    for name, a, b in (("q", q0, q1), ("k", k0, k1), ("v", v0, v1), ("output2", o20, o21)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name
    written = q1[:, :sum(Ms)]
    assert torch.isfinite(written.float()).all() and torch.isnan(q1[:, sum(Ms):].float()).all()


def test_qkv_epilogue_rejects_bad_arguments(dev):
    import torch
    from llmr_amd import capi, ops
    g = ops.default_graph()
    H, K, M = 2, 256, 64
    w = _weight(320, 12, 3 * H * 128 + 256, K, dev)
    x = ops.Tensor.from_torch(_x(321, M, K, 30, dev))
    q = torch.empty(H, M, 128, dtype=torch.float16, device=dev)
    k, v = torch.empty_like(q), torch.empty_like(q)
    heads = ops.QkvHeads(q, k, v, H, [(None, None, 0)])
    cases = [
        (3 * H * 128 + 256, STORE, 0, heads, "out_dim"),                                # STORE: out_dim != 3 H 128
        (3 * H * 128, capi.EPI_GATED_RESIDUAL, 0, heads, "GATED_RESIDUAL"),
        (3 * H * 128 + 256, GELU, 256, heads, "split"),                                 # split != 3 H 128
        (3 * H * 128, STORE, 0, ops.QkvHeads(q, k, v, H, [(None, None, 1)]), "row0"),   # past seq_len
    ]
    for N, epi, split, h, what in cases:
        y2 = torch.empty(M, N - split, dtype=torch.bfloat16, device=dev) if epi == GELU else None
        gate = torch.ones(N, device=dev) if epi == capi.EPI_GATED_RESIDUAL else None
        out = torch.empty(M, N, device=dev) if epi == capi.EPI_GATED_RESIDUAL else None
        job = ops.MatmulJob(w, x, out, M, 0, gate, y2)
        with pytest.raises(capi.LlmrError, match=what):
            ops.dispatch_batch_matmul_multi(g, [job], N, K, epi, split, heads=h)
    torch.cuda.synchronize()
