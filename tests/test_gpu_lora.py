"""GPU LoRA (llmr_lora_correction, llmr_batch_matmul_lora, llmr_q8_lora_merge)
vs the oracle: bit-identical (the kernels form every f32 sum in the
reference's order, without contraction), except llmr_batch_matmul_lora on
the two-pass GEMM, which merges the adapter into its 16-bit weight image and
is held to the GEMM's tolerance."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _lora(dev, r, rank, in_dim, b_total, scale, std=0.05):
    import torch
    from llmr_amd import ops
    A = (std * r.standard_normal((rank, in_dim))).astype(np.float32)
    B = (std * r.standard_normal((b_total, rank))).astype(np.float32)
    return A, B, ops.LoraTensor(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), rank, scale)


def _act(x_f32, xtype, dev):
    import torch
    t = torch.from_numpy(x_f32)
    t = {0: t, 1: t.half(), 30: t.bfloat16()}[xtype]
    return t.to(dev)


@pytest.mark.parametrize("seq,in_dim,rank,out_dim,b_rows,row_off,w_off,xtype", [
    (37, 512, 8, 300, 200, 50, 30, 0),      # f32 input, sub-range of a wider output
    (64, 3072, 32, 3072, 0, 0, 0, 30),      # Flux dim, bf16 input, whole output
    (5, 768, 48, 1024, 256, 768, 512, 1),   # f16 input, one slot of a fused Q|K|V adapter
    (3, 256, 256, 260, 0, 0, 0, 0),         # the largest rank
    (17, 700, 1, 129, 0, 0, 0, 30),         # rank 1, ragged sizes
    (300, 512, 16, 3072, 2000, 512, 100, 30),  # rank 16: the register-resident hop 2 over 3 token spans
    (129, 256, 4, 520, 0, 0, 0, 1),         # rank 4, ragged columns and tokens
])
def test_lora_correction_bit_exact(orc, dev, seq, in_dim, rank, out_dim, b_rows, row_off, w_off, xtype):
    import torch
    from llmr_amd import ops
    r = np.random.default_rng(seq * 1000 + rank)
    rows = b_rows or out_dim
    A, B, lora = _lora(dev, r, rank, in_dim, w_off + rows + 3, 0.8)
    x = r.standard_normal((seq, in_dim)).astype(np.float32)
    xt = _act(x, xtype, dev)
    y0 = r.standard_normal((seq, out_dim)).astype(np.float32)
    y = torch.from_numpy(y0).to(dev)
    scratch = torch.empty(seq * rank, device=dev)
    g = ops.default_graph()
    ops.dispatch_lora_correction(g, lora, scratch, ops.Tensor.from_torch(xt), ops.Tensor.from_torch(y), in_dim,
                                 out_dim, seq, b_rows, row_off, w_off)
    torch.cuda.synchronize()
    xf = xt.float().cpu().numpy()
    s_ref = orc.lora_down(A, xf)
    np.testing.assert_array_equal(scratch.cpu().numpy().reshape(seq, rank), s_ref)
    y_ref = orc.lora_up(B, s_ref, y0, 0.8, row_offset=row_off, weight_row_offset=w_off, b_rows=rows)
    np.testing.assert_array_equal(y.cpu().numpy(), y_ref)


def test_batch_matmul_with_lora_equals_base_plus_correction(orc, dev):
    """dispatch_batch_matmul with an adapter = the plain GEMM, then the
    correction on its output (dit.c3:1299-1300), at the Flux img_attn.qkv K
    slot: base rows [dim, 2 dim) of the fused weight, adapter rows likewise."""
    import torch
    from llmr_amd import glue, ops
    d, seq, rank = 3072, 300, 16
    r = np.random.default_rng(11)
    w = glue.synth_q4k(3 * d, d, 321, device=dev)
    A, B, lora = _lora(dev, r, rank, d, 3 * d, 1.25)
    x = torch.randn(seq, d, device=dev).bfloat16()
    g = ops.default_graph()
    wt = ops.Tensor.quantized(w, 12, 3 * d, d)
    base = torch.empty(seq, d, device=dev)
    ops.dispatch_batch_matmul(g, wt, ops.Tensor.from_torch(x), ops.Tensor.from_torch(base), d, d, seq, d)
    y = torch.empty(seq, d, device=dev)
    scratch = torch.empty(seq * rank, device=dev)
    ops.dispatch_batch_matmul(g, wt, ops.Tensor.from_torch(x), ops.Tensor.from_torch(y), d, d, seq, d,
                              lora=lora, lora_scratch=scratch, lora_weight_row_offset=d)
    torch.cuda.synchronize()
    s_ref = orc.lora_down(A, x.float().cpu().numpy())
    y_ref = orc.lora_up(B, s_ref, base.cpu().numpy(), 1.25, weight_row_offset=d, b_rows=d)
    np.testing.assert_array_equal(y.cpu().numpy(), y_ref)
    # a merged-away adapter (present False) leaves the plain GEMM
    lora.present = False
    ops.dispatch_batch_matmul(g, wt, ops.Tensor.from_torch(x), ops.Tensor.from_torch(y), d, d, seq, d,
                              lora=lora, lora_scratch=scratch)
    torch.cuda.synchronize()
    assert torch.equal(y, base)


@pytest.mark.parametrize("rows,in_dim,rank,off,b_rows", [
    (12, 512, 4, 0, 12),
    (40, 3072, 32, 9, 25),
    (8, 256, 256, 3, 5),
    (6, 768, 1, 0, 6),
])
def test_q8_lora_merge_bit_exact(orc, dev, rows, in_dim, rank, off, b_rows):
    import torch
    from llmr_amd import gguf, ops
    r = np.random.default_rng(rows + rank)
    w = gguf.quantize((0.05 * r.standard_normal((rows, in_dim))).astype(np.float32), gguf.GGML_Q8_0)
    A, B, lora = _lora(dev, r, rank, in_dim, b_rows, 0.6, std=0.2)
    wd = torch.from_numpy(w.copy()).to(dev)
    g = ops.default_graph()
    assert ops.merge_one_site(g, ops.Tensor.quantized(wd, gguf.GGML_Q8_0, rows, in_dim), lora, off)
    torch.cuda.synchronize()
    assert not lora.present
    np.testing.assert_array_equal(wd.cpu().numpy(), orc.q8_lora_merge(w, A, B, in_dim, 0.6, dst_row_offset=off))


def test_lora_rejects_and_skips(dev):
    import torch
    from llmr_amd import capi, glue, gguf, ops
    g = ops.default_graph()
    r = np.random.default_rng(3)
    # in_dim % 256 != 0: the merge is not taken (the reference skips it)
    w = torch.zeros(4 * 96 // 32 * 34, dtype=torch.uint8, device=dev)
    _, _, lora = _lora(dev, r, 4, 96, 4, 1.0)
    assert not ops.merge_one_site(g, ops.Tensor.quantized(w, gguf.GGML_Q8_0, 4, 96), lora)
    assert lora.present
    with pytest.raises(capi.LlmrError):
        g.ctx.q8_lora_merge(w.data_ptr(), lora.a.data_ptr(), lora.b.data_ptr(), 96, 4, 0, 4, 1.0)
    # a Q4_K base keeps the runtime correction
    wq = glue.synth_q4k(8, 256, 1, device=dev)
    _, _, l2 = _lora(dev, r, 4, 256, 8, 1.0)
    assert not ops.merge_one_site(g, ops.Tensor.quantized(wq, 12, 8, 256), l2)
    # rank > 256: the correction leaves the output as it is
    x = torch.randn(4, 256, device=dev)
    y = torch.randn(4, 64, device=dev)
    y0 = y.clone()
    big = ops.LoraTensor(torch.zeros(300, 256, device=dev), torch.zeros(64, 300, device=dev), 300, 1.0)
    scratch = torch.empty(4 * 300, device=dev)
    ops.dispatch_lora_correction(g, big, scratch, ops.Tensor.from_torch(x), ops.Tensor.from_torch(y), 256, 64, 4)
    torch.cuda.synchronize()
    assert torch.equal(y, y0)
    # row_offset + b_rows beyond out_dim is an argument error
    _, _, l3 = _lora(dev, r, 4, 256, 64, 1.0)
    with pytest.raises(capi.LlmrError):
        g.ctx.lora_correction(l3.c_struct(), scratch.data_ptr(), x.data_ptr(), 0, y.data_ptr(), 256, 64, 4, 40, 30)


def _split_bf16(x):
    from llmr_amd.workloads import round_bf16
    hi = round_bf16(x)
    return hi, round_bf16((x - hi).astype(np.float32))


def _merged_rows(orc, blk, xs16, A, B, scale, rows_s, N, K, row_off, w_off, b_rows, ot):
    """Sampled output rows of x . W'^T in f64, W' the 16-bit weight image
    with the adapter merged: W16 + d on the slot's features, d = (scale B) A
    with both factors split into bf16 hi + lo parts and summed as hi hi +
    hi lo + lo hi (exactly here, rounded to f32 once), added to W16 in f32
    and rounded to the operand type once more (nearest even)."""
    from llmr_amd.workloads import round_bf16
    if ot == 1:
        w16 = orc.f16_to_f32(orc.dequant_q4k_operand(blk)).reshape(N, K)
    else:
        w16 = round_bf16(orc.dequant_q4k(blk)).reshape(N, K)
    bs = np.float32(scale) * B[w_off:w_off + b_rows]  # [b_rows, rank], f32 products
    bh, bl = (t.astype(np.float64) for t in _split_bf16(bs))
    ah, al = (t.astype(np.float64) for t in _split_bf16(A))
    dlt = (bh @ ah + bh @ al + bl @ ah).astype(np.float32)
    merged = w16.copy()
    s = w16[row_off:row_off + b_rows] + dlt
    merged[row_off:row_off + b_rows] = (s.astype(np.float16).astype(np.float32) if ot == 1 else round_bf16(s))
    return xs16[rows_s].astype(np.float64) @ merged.T.astype(np.float64)


# GEMMs on the two-pass kernel (>= 2048 tokens, >= 128 tiles of 256 x 256)
# with rank <= 64 merge the adapter into the 16-bit weight image as it is
# built: W' = RN16(W16 + d) on the slot's features, d = (scale B) A on the
# matrix cores from bf16 hi/lo splits of both factors. Features outside
# the slot equal the plain GEMM bit for bit (their image is untouched); the
# slot equals x . W'^T to f32 accumulation order (checked against an exact
# host model of W'), GEMM + exact correction within the 16-bit rounding of
# W', and the oracle (the reference's f32 correction after the GEMM) within
# the GEMM bar.
@pytest.mark.parametrize("M,N,K,rank,b_rows,row_off,w_off,xtype", [
    (2304, 4096, 512, 16, 1024, 512, 64, 30),    # bf16, a slot of the output
    (2400, 4100, 768, 48, 0, 0, 0, 1),           # f16, whole output, ragged M and N
    (2048, 4096, 512, 64, 2000, 100, 7, 0),      # f32 input (rounded to bf16 first: Q4_K), the largest merged rank
])
def test_batch_matmul_lora_fused(orc, dev, M, N, K, rank, b_rows, row_off, w_off, xtype):
    import torch
    from llmr_amd import gguf, ops, synth
    from conftest import rel_l2
    r = np.random.default_rng(M + rank)
    rows = b_rows or N
    A, B, lora = _lora(dev, r, rank, K, w_off + rows + 5, 0.7)
    blk = gguf.quantize(synth.normal(17, 2, N * K, 0.02), gguf.GGML_Q4_K)
    wt = ops.Tensor.quantized(torch.from_numpy(blk).to(dev), gguf.GGML_Q4_K, N, K)
    xt = _act(synth.normal(17, 1, M * K).reshape(M, K), xtype, dev)
    g = ops.default_graph()
    base = torch.empty(M, N, device=dev)
    ops.dispatch_batch_matmul(g, wt, ops.Tensor.from_torch(xt), ops.Tensor.from_torch(base), N, K, M, 0)
    fused = torch.empty(M, N, device=dev)
    scratch = torch.empty(M * rank, device=dev)
    ops.dispatch_batch_matmul(g, wt, ops.Tensor.from_torch(xt), ops.Tensor.from_torch(fused), N, K, M, 0,
                              lora=lora, lora_scratch=scratch, lora_b_rows=b_rows, lora_row_offset=row_off,
                              lora_weight_row_offset=w_off)
    again = torch.empty(M, N, device=dev)
    ops.dispatch_batch_matmul(g, wt, ops.Tensor.from_torch(xt), ops.Tensor.from_torch(again), N, K, M, 0,
                              lora=lora, lora_scratch=scratch, lora_b_rows=b_rows, lora_row_offset=row_off,
                              lora_weight_row_offset=w_off)
    exact = base.clone()
    ops.dispatch_lora_correction(g, lora, scratch, ops.Tensor.from_torch(xt), ops.Tensor.from_torch(exact), K, N,
                                 M, b_rows, row_off, w_off)
    torch.cuda.synchronize()
    assert torch.equal(fused, again)  # deterministic
    f, e, b0 = fused.cpu().numpy(), exact.cpu().numpy(), base.cpu().numpy()
    slot = slice(row_off, row_off + rows)
    outside = np.ones(N, bool)
    outside[slot] = False
    assert np.array_equal(f[:, outside], b0[:, outside])
    err = rel_l2(f[:, slot], e[:, slot])
    rows_s = np.array([0, 1, M // 2, M - 1], np.int64)
    xs = xt.float().cpu().numpy()
    # f32 activations against Q4_K weights become bf16 operands (as bf16 ones)
    bf = xtype in (0, 30)
    xs16 = torch.from_numpy(xs).bfloat16().float().numpy() if xtype == 0 else xs
    model = _merged_rows(orc, blk, xs16, A, B, 0.7, rows_s, N, K, row_off, w_off, rows, 30 if bf else 1)
    err_model = rel_l2(f[rows_s], model)
    print(f"M={M} N={N} K={K} rank={rank}: vs merged-image model {err_model:.2e}, vs GEMM + correction {err:.2e}")
    assert err_model <= 2e-5
    assert err <= (5e-3 if bf else 1e-3)
    ref = orc.batch_matmul(blk, gguf.GGML_Q4_K, xs, N, K, M, 0, rows=rows_s.astype(np.uint32))
    s_ref = orc.lora_down(A, xs[rows_s])
    ref = orc.lora_up(B, s_ref, ref, 0.7, row_offset=row_off, weight_row_offset=w_off, b_rows=rows)
    assert rel_l2(f[rows_s], ref) <= 1e-2
