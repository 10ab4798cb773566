"""Block-glue entry points (C-ABI through llmr_amd.glue) vs the oracle's
per-dispatch restatements.

Tolerances: f32 outputs differ from the oracle only by reduction order and
transcendental ulps (rtol 1e-5); 16-bit outputs are the f32 value rounded once,
so they must sit within half an ulp of the 16-bit type of the oracle's value
plus that f32 slack."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ULP = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _close(got: torch.Tensor, ref: np.ndarray, dtype, atol=1e-6):
    g = got.float().cpu().numpy()
    tol = (0.5 * ULP[dtype] + 1e-5) * np.abs(ref) + atol
    bad = np.abs(g - ref) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance; max err {np.abs(g - ref).max()}"


def _rng(seed):
    return np.random.default_rng(seed)


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim,rows", [(3840, 37), (3072, 5), (100, 9)])
def test_rmsnorm_modulate(orc, dev, dtype, dim, rows):
    from llmr_amd import glue
    r = _rng(dim + rows)
    xf = r.standard_normal((rows, dim + 12)).astype(np.float32)  # rows of a wider buffer
    w = (1 + 0.1 * r.standard_normal(dim)).astype(np.float32)
    sc = (0.5 * r.standard_normal(dim)).astype(np.float32)
    x_t = _dev(xf, dev)[:, :dim]
    out = torch.empty(rows, dim, dtype=dtype, device=dev)
    glue.batch_rmsnorm(x_t, _dev(w, dev), out, 1e-5, mod_scale=_dev(sc, dev))
    torch.cuda.synchronize()
    ref = orc.modulate(orc.batch_rmsnorm(xf[:, :dim], w, 1e-5), sc)
    _close(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layernorm_adaln_on_row_range(orc, dev, dtype):
    from llmr_amd import glue
    r = _rng(11)
    S, nt, dim = 303, 44, 3072  # 259 rows: a workgroup of four rows is part-filled
    h = (r.standard_normal((S, dim)) * 3 + 1.5).astype(np.float32)
    sc = (0.3 * r.standard_normal(dim)).astype(np.float32)
    sh = (0.3 * r.standard_normal(dim)).astype(np.float32)
    h_t = _dev(h, dev)
    out = torch.full((S, dim), 7.0, dtype=dtype, device=dev)
    glue.batch_layernorm(h_t[nt:], out[nt:], 1e-6, mod_scale=_dev(sc, dev), mod_shift=_dev(sh, dev))
    torch.cuda.synchronize()
    ref = orc.modulate(orc.batch_layernorm(h[nt:], 1e-6), sc, sh)
    _close(out[nt:], ref, dtype, atol=1e-5)
    assert (out[:nt].float() == 7.0).all()  # rows outside the range untouched


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layernorm_split_equals_two_calls(orc, dev, dtype):
    """llmr_batch_layernorm_split (the Flux double block's text and image
    LayerNorms in one launch): rows below split_row with the first
    modulation pair, the rest with the second (here scale only, no shift),
    bit for bit the two batch_layernorm calls, and the oracle's LayerNorm +
    modulation; a split_row that is not a multiple of 4, or past n_rows, is
    refused."""
    from llmr_amd import capi, glue
    r = _rng(13)
    S, nt, dim = 303, 44, 3072  # 259 image rows: the last workgroup of four rows is part-filled
    h = (r.standard_normal((S, dim)) * 3 + 1.5).astype(np.float32)
    sc, sh, sc2 = ((0.3 * r.standard_normal(dim)).astype(np.float32) for _ in range(3))
    h_t = _dev(h, dev)
    one = torch.full((S, dim), 7.0, dtype=dtype, device=dev)
    two = torch.full((S, dim), 7.0, dtype=dtype, device=dev)
    glue.batch_layernorm_split(h_t, one, 1e-6, nt, (_dev(sc, dev), _dev(sh, dev)), (_dev(sc2, dev), None))
    glue.batch_layernorm(h_t[:nt], two[:nt], 1e-6, mod_scale=_dev(sc, dev), mod_shift=_dev(sh, dev))
    glue.batch_layernorm(h_t[nt:], two[nt:], 1e-6, mod_scale=_dev(sc2, dev))
    torch.cuda.synchronize()
    assert torch.equal(one, two)
    _close(one[:nt], orc.modulate(orc.batch_layernorm(h[:nt], 1e-6), sc, sh), dtype, atol=1e-5)
    _close(one[nt:], orc.modulate(orc.batch_layernorm(h[nt:], 1e-6), sc2), dtype, atol=1e-5)
    for bad in (nt + 2, S + 4):
        with pytest.raises(capi.LlmrError, match="split_row"):
            glue.batch_layernorm_split(h_t, one, 1e-6, bad, (None, None), (None, None))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_qkv_heads_joint_rows(orc, dev, dtype):
    """Image rows of a linear1-shaped buffer (stride > 3*H*128) into rows
    row0.. of the joint Q/K/V, with head norm and RoPE; V unrotated."""
    from llmr_amd import glue, workloads
    r = _rng(12)
    H, S, row0, rows, extra = 3, 70, 20, 50, 256
    src = r.standard_normal((rows, 3 * H * 128 + extra)).astype(np.float32)
    qn = (1 + 0.1 * r.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * r.standard_normal(128)).astype(np.float32)
    att = workloads.Attention("t", H, S, 128, 6, 8, 8, (16, 56, 56), 10000.0)
    cos_t, sin_t = workloads.rope_tables(workloads.attention_positions(att), att.axes, att.theta)
    q = torch.zeros(H, S, 128, dtype=dtype, device=dev)
    k = torch.zeros_like(q)
    v = torch.zeros_like(q)
    glue.qkv_heads(_dev(src, dev), H, q, k, v, row0, _dev(qn, dev), _dev(kn, dev), 1e-6,
                   (_dev(cos_t, dev), _dev(sin_t, dev)))
    torch.cuda.synchronize()
    D = H * 128
    sl = slice(row0, row0 + rows)
    rq = orc.rope_apply(orc.transpose_heads(orc.batch_head_norm(src[:, :D], qn, H, 1e-6), H), cos_t[sl], sin_t[sl])
    rk = orc.rope_apply(orc.transpose_heads(orc.batch_head_norm(src[:, D:2 * D], kn, H, 1e-6), H), cos_t[sl],
                        sin_t[sl])
    rv = orc.transpose_heads(src[:, 2 * D:3 * D], H)
    _close(q[:, sl], rq, dtype, atol=1e-5)
    _close(k[:, sl], rk, dtype, atol=1e-5)
    _close(v[:, sl], rv, dtype)
    assert (q[:, :row0].float() == 0).all() and (v[:, row0 + rows:].float() == 0).all()


def test_qkv_heads_plain_transpose(orc, dev):
    from llmr_amd import glue
    r = _rng(13)
    H, S = 2, 33
    src = r.standard_normal((S, 3 * H * 128)).astype(np.float32)
    q = torch.empty(H, S, 128, dtype=torch.float32, device=dev)
    k, v = torch.empty_like(q), torch.empty_like(q)
    glue.qkv_heads(_dev(src, dev), H, q, k, v)
    torch.cuda.synchronize()
    for i, t in enumerate((q, k, v)):
        np.testing.assert_array_equal(t.cpu().numpy(), orc.transpose_heads(src[:, i * H * 128:(i + 1) * H * 128], H))


@pytest.mark.parametrize("mode,norm", [(2, True), (1, False), (0, False), (2, False)])
def test_gated_residual_modes(orc, dev, mode, norm):
    from llmr_amd import glue
    r = _rng(14 + mode)
    S, nt, dim = 203, 40, 3840  # 163 rows: a workgroup of four rows is part-filled
    h = r.standard_normal((S, dim)).astype(np.float32)
    x = r.standard_normal((S - nt, dim)).astype(np.float32) * 2
    gate = r.standard_normal(dim).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(dim)).astype(np.float32)
    h_t = _dev(h, dev)
    glue.gated_residual(h_t[nt:], _dev(x, dev), _dev(gate, dev) if mode else None, mode,
                        _dev(nw, dev) if norm else None, 1e-5)
    torch.cuda.synchronize()
    y = orc.batch_rmsnorm(x, nw, 1e-5) if norm else x
    if mode == 0:
        ref = h[nt:] + y
    else:
        ref = orc.gated_residual(h[nt:], gate, y, mode == 2)
    got = h_t.cpu().numpy()
    np.testing.assert_allclose(got[nt:], ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(got[:nt], h[:nt])


@pytest.mark.parametrize("mode,norm,dim,dtype,shift", [
    (2, True, 3840, torch.bfloat16, False),   # the Z-Image block's form (scale only)
    (1, False, 1000, torch.float16, True),    # a ragged width (NV 4), linear gate, scale and shift
    (0, True, 2048, torch.float32, False),    # plain add
])
def test_gated_residual_rmsnorm_equals_two_calls(orc, dev, mode, norm, dim, dtype, shift):
    """llmr_gated_residual_rmsnorm: the residual update and the updated rows'
    RMSNorm + modulation in one pass, bit for bit gated_residual followed by
    batch_rmsnorm (both outputs: the residual and the normalized rows), and
    the oracle's RMSNorm + modulation of the updated rows; a dim above 4096
    is refused."""
    from llmr_amd import capi, glue
    r = _rng(30 + mode)
    S, nt = 203, 40  # 163 rows: a workgroup of four rows is part-filled
    h = r.standard_normal((S, dim)).astype(np.float32)
    x = r.standard_normal((S - nt, dim)).astype(np.float32) * 2
    gate = r.standard_normal(dim).astype(np.float32)
    nw, fw = ((1 + 0.1 * r.standard_normal(dim)).astype(np.float32) for _ in range(2))
    sc, sh = ((0.3 * r.standard_normal(dim)).astype(np.float32) for _ in range(2))
    ha, hb = _dev(h, dev), _dev(h, dev)
    oa = torch.full((S - nt, dim), 7.0, dtype=dtype, device=dev)
    ob = torch.full((S - nt, dim), 7.0, dtype=dtype, device=dev)
    gt = _dev(gate, dev) if mode else None
    nwt = _dev(nw, dev) if norm else None
    sht = _dev(sh, dev) if shift else None
    glue.gated_residual_rmsnorm(ha[nt:], _dev(x, dev), gt, mode, nwt, 1e-5, _dev(fw, dev), oa, 1e-6,
                                mod_scale=_dev(sc, dev), mod_shift=sht)
    glue.gated_residual(hb[nt:], _dev(x, dev), gt, mode, nwt, 1e-5)
    glue.batch_rmsnorm(hb[nt:], _dev(fw, dev), ob, 1e-6, mod_scale=_dev(sc, dev), mod_shift=sht)
    torch.cuda.synchronize()
    assert torch.equal(ha, hb) and torch.equal(oa, ob)
    h1 = ha[nt:].cpu().numpy()
    ref = orc.modulate(orc.batch_rmsnorm(h1, fw, 1e-6), sc, sh if shift else None)
    _close(oa, ref, dtype, atol=1e-5)
    np.testing.assert_array_equal(ha[:nt].cpu().numpy(), h[:nt])
    with pytest.raises(capi.LlmrError, match="4096"):
        w = torch.zeros(4, 4104, device=dev)
        glue.gated_residual_rmsnorm(w, w, None, 0, None, 1e-5, w[0], torch.zeros_like(w), 1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_activation_concat_gelu_silu_mul(orc, dev, dtype):
    """The single-stream concat: attention output -> cat[:, :d], gelu(linear1
    MLP half) -> cat[:, d:]; and silu(gate) * up from one buffer."""
    from llmr_amd import capi, glue
    r = _rng(15)
    S, d, m = 65, 256, 512
    o = r.standard_normal((S, d)).astype(np.float32)
    l1 = (3 * r.standard_normal((S, 3 * d + m))).astype(np.float32)
    l1_t = _dev(l1, dev)
    cat = torch.empty(S, d + m, dtype=dtype, device=dev)
    glue.activation(_dev(o, dev), cat[:, :d], capi.ACT_COPY)
    glue.activation(l1_t[:, 3 * d:], cat[:, d:], capi.ACT_GELU_TANH)
    gu = (3 * r.standard_normal((S, 2 * m))).astype(np.float32)
    gu_t = _dev(gu, dev)
    sm = torch.empty(S, m, dtype=dtype, device=dev)
    glue.activation(gu_t[:, :m], sm, capi.ACT_SILU_MUL, src2=gu_t[:, m:])
    torch.cuda.synchronize()
    _close(cat[:, :d], o, dtype)
    _close(cat[:, d:], orc.gelu(l1[:, 3 * d:]), dtype, atol=1e-6)
    _close(sm, orc.silu(gu[:, :m]) * gu[:, m:], dtype, atol=1e-6)


def test_activation_in_place_single_row(orc, dev):
    from llmr_amd import capi, glue
    x = np.linspace(-9, 9, 3072, dtype=np.float32)[None, :]
    t = _dev(x, dev)
    glue.activation(t, t, capi.ACT_SILU)
    torch.cuda.synchronize()
    np.testing.assert_allclose(t.cpu().numpy(), orc.silu(x), rtol=1e-6, atol=1e-7)


def test_timestep_patchify_unpatchify(orc, dev):
    from llmr_amd import glue
    emb = torch.empty(256, dtype=torch.float32, device=dev)
    glue.timestep_embed(emb, 500.0)
    r = _rng(16)
    lat = r.standard_normal((16, 32, 48)).astype(np.float32)
    p = torch.empty(16 * 24, 64, dtype=torch.bfloat16, device=dev)
    glue.patchify(_dev(lat, dev), p, 2)
    pf = _dev(orc.patchify(lat, 2), dev)
    back = torch.empty(16, 32, 48, dtype=torch.float32, device=dev)
    glue.unpatchify(pf, back, 2)
    torch.cuda.synchronize()
    # freq = exp(...) may differ by an ulp between device and host exp; the
    # angle t * freq then moves by up to t * ulp(1) = 500 * 1.2e-7 = 6e-5
    np.testing.assert_allclose(emb.cpu().numpy(), orc.timestep_embed(256, 500.0), rtol=0, atol=1.5e-4)
    _close(p, orc.patchify(lat, 2), torch.bfloat16)
    np.testing.assert_array_equal(back.cpu().numpy(), lat)


def test_glue_rejects_bad_arguments(dev):
    from llmr_amd import capi, glue
    x = torch.zeros(4, 8192 + 4, device=dev)
    out = torch.zeros(4, 8192 + 4, device=dev)
    w = torch.ones(8192 + 4, device=dev)
    with pytest.raises(capi.LlmrError) as e:  # wider than the register-resident row
        glue.batch_rmsnorm(x, w, out, 1e-5)
    assert e.value.code == capi.LLMR_ERR_INVALID_ARG
    x = torch.zeros(4, 130, device=dev)
    with pytest.raises(capi.LlmrError):  # dim % 4 != 0
        glue.batch_rmsnorm(x[:, :126], w, torch.zeros(4, 126, device=dev), 1e-5)
    ctx = glue.default_graph().ctx
    base = torch.zeros(64, device=dev)
    with pytest.raises(capi.LlmrError):  # misaligned pointer
        ctx.gated_residual(base.data_ptr() + 4, 8, base.data_ptr(), 8, None, None, 0, 8, 2, 1e-5)
    with pytest.raises(capi.LlmrError):  # row0 + rows beyond the sequence
        q = torch.zeros(1, 8, 128, device=dev, dtype=torch.float16)
        glue.qkv_heads(torch.zeros(8, 384, device=dev), 1, q, q.clone(), q.clone(), row0=1)
    with pytest.raises(capi.LlmrError):  # destination columns beyond its stride
        ctx.activation(base.data_ptr(), 8, 0, 0, base.data_ptr(), 0, 8, 4, 2, 8, capi.ACT_COPY)


def test_synth_q4k_matches_host_quantizer(dev):
    """The device generator + quantizer is byte-identical to the package's host
    path (synth.normal + gguf.quantize_q4k) on the same stream."""
    from llmr_amd import glue, gguf, synth
    rows, K, stream = 96, 768, 4242
    blk = glue.synth_q4k(rows, K, stream, 0.02, seed=42, device=dev)
    torch.cuda.synchronize()
    host = gguf.quantize_q4k(synth.normal(42, stream, rows * K, 0.02).reshape(rows, K))
    got = blk.cpu().numpy()
    assert got.size == host.size
    diff = np.flatnonzero(got != host)
    assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:8]}"


def test_synth_q4k_distribution(orc, dev):
    from llmr_amd import glue
    rows, K = 1024, 3072
    blk = glue.synth_q4k(rows, K, 77, 0.02, device=dev)
    torch.cuda.synchronize()
    w = orc.dequant_q4k(blk.cpu().numpy())
    assert np.isfinite(w).all()
    assert abs(w.mean()) < 1e-4 and abs(w.std() / 0.02 - 1) < 0.02


def test_glue_fusions_random(dev):
    """Twelve seeded random cases each of the split LayerNorm (split_row a
    multiple of 4 up to n_rows, width up to 8192) and the fused residual +
    RMSNorm (width up to 4096, every gate mode, with and without the
    post-norm, scale and shift present or not), against their two-call
    forms bit for bit, over ragged row counts and output types."""
    import random
    from llmr_amd import glue
    rnd = random.Random(1203)
    r = _rng(40)
    dts = (torch.float32, torch.float16, torch.bfloat16)
    for case in range(12):
        dim, rows = 4 * rnd.randint(1, 2048), rnd.randint(1, 700)
        split = 4 * rnd.randint(0, rows // 4)
        dt = rnd.choice(dts)
        h = _dev((r.standard_normal((rows, dim)) * 2 + 0.5).astype(np.float32), dev)
        vecs = [_dev((0.3 * r.standard_normal(dim)).astype(np.float32), dev) if rnd.random() < 0.7 else None
                for _ in range(4)]
        a = torch.full((rows, dim), 7.0, dtype=dt, device=dev)
        b = torch.full((rows, dim), 7.0, dtype=dt, device=dev)
        print(f"split layernorm case {case}: rows {rows} dim {dim} split {split} {dt}", flush=True)
        glue.batch_layernorm_split(h, a, 1e-6, split, (vecs[0], vecs[1]), (vecs[2], vecs[3]))
        if split:
            glue.batch_layernorm(h[:split], b[:split], 1e-6, mod_scale=vecs[0], mod_shift=vecs[1])
        if split < rows:
            glue.batch_layernorm(h[split:], b[split:], 1e-6, mod_scale=vecs[2], mod_shift=vecs[3])
        torch.cuda.synchronize()
        assert torch.equal(a, b), case
    for case in range(12):
        dim, rows = 4 * rnd.randint(1, 1024), rnd.randint(1, 700)
        mode, norm = rnd.randint(0, 2), rnd.random() < 0.5
        dt = rnd.choice(dts)
        h = r.standard_normal((rows, dim)).astype(np.float32)
        x = _dev((2 * r.standard_normal((rows, dim))).astype(np.float32), dev)
        gate = _dev(r.standard_normal(dim).astype(np.float32), dev) if mode else None
        nw, fw = (_dev((1 + 0.1 * r.standard_normal(dim)).astype(np.float32), dev) for _ in range(2))
        sc = _dev((0.3 * r.standard_normal(dim)).astype(np.float32), dev) if rnd.random() < 0.7 else None
        sh = _dev((0.3 * r.standard_normal(dim)).astype(np.float32), dev) if rnd.random() < 0.5 else None
        ha, hb = _dev(h, dev), _dev(h, dev)
        oa = torch.full((rows, dim), 7.0, dtype=dt, device=dev)
        ob = torch.full((rows, dim), 7.0, dtype=dt, device=dev)
        print(f"residual rmsnorm case {case}: rows {rows} dim {dim} mode {mode} norm {norm} {dt}", flush=True)
        glue.gated_residual_rmsnorm(ha, x, gate, mode, nw if norm else None, 1e-5, fw, oa, 1e-6, mod_scale=sc,
                                    mod_shift=sh)
        glue.gated_residual(hb, x, gate, mode, nw if norm else None, 1e-5)
        glue.batch_rmsnorm(hb, fw, ob, 1e-6, mod_scale=sc, mod_shift=sh)
        torch.cuda.synchronize()
        assert torch.equal(ha, hb) and torch.equal(oa, ob), case
