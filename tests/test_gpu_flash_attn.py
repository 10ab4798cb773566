"""GPU flash attention vs the oracle (relative L2 <= 1e-2; the oracle restates
flash_attention_v2) plus size-independent properties."""
import math

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _to_dev(a, xtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    t = {0: t, 1: t.to(torch.float16), 30: t.to(torch.bfloat16)}[xtype]
    return t.to(dev)


def _fa(dev, q, k, v, xtype, scale=None):
    import torch
    from llmr_amd import ops
    qt, kt, vt = (_to_dev(a, xtype, dev) for a in (q, k, v))
    o = ops.flash_attention(qt, kt, vt, scale)
    torch.cuda.synchronize()
    back = [t.to(torch.float32).cpu().numpy() for t in (qt, kt, vt)]
    return o.cpu().numpy(), back


# f16 inputs take the 64-query-per-wave kernel: sequence lengths cover a
# partial last tile at each position relative to its 3-tile unroll (the
# masked loop copy starting in the first, second or third body position),
# S < 64, S = 64, and a whole-tile end (S = 4352: one padding tile).
@pytest.mark.parametrize("H,S,xtype", [(2, 200, 1), (1, 64, 1), (1, 1, 1), (3, 63, 0), (2, 129, 30),
                                       (1, 257, 0), (4, 512, 1), (2, 1000, 30), (1, 65, 1), (2, 257, 1),
                                       (1, 383, 1), (3, 1000, 1), (2, 1089, 1), (1, 4352, 1)])
def test_fa_parity_small(orc, dev, H, S, xtype):
    from llmr_amd import synth
    n = H * S * 128
    q = synth.normal(1, 3, n).reshape(H, S, 128)
    k = synth.normal(1, 4, n).reshape(H, S, 128)
    v = synth.normal(1, 5, n).reshape(H, S, 128)
    o, (qr, kr, vr) = _fa(dev, q, k, v, xtype)
    ref = orc.flash_attention(qr, kr, vr, 1.0 / math.sqrt(128))
    err = rel_l2(o, ref)
    print(f"H={H} S={S} xtype={xtype}: rel_l2={err:.3e}")
    assert np.all(np.isfinite(o))
    assert err <= TOL


@pytest.mark.parametrize("xtype", [1, 0])
def test_fa_large_scores(orc, dev, xtype):
    """Scores of magnitude ~100 (scaled Q and K): the running max is raised
    many times along the keys, exercising the lazy rescaling of O and l."""
    from llmr_amd import synth
    H, S = 2, 700
    n = H * S * 128
    q = synth.normal(6, 3, n).reshape(H, S, 128) * 3
    k = synth.normal(6, 4, n).reshape(H, S, 128) * 3
    v = synth.normal(6, 5, n).reshape(H, S, 128)
    o, (qr, kr, vr) = _fa(dev, q, k, v, xtype)
    ref = orc.flash_attention(qr, kr, vr, 1.0 / math.sqrt(128))
    err = rel_l2(o, ref)
    print(f"large scores xtype={xtype}: rel_l2={err:.3e}")
    assert np.all(np.isfinite(o))
    assert err <= TOL


@pytest.mark.parametrize("H,S,xtype", [(5, 700, 0), (24, 4608, 0), (2, 300, 30), (7, 129, 30)])
def test_fa_wide_inputs_match_fp16_inputs(dev, H, S, xtype):
    """f32 / bf16 Q, K, V are rounded to fp16 where the kernel reads them (K and
    V by a conversion pass into the workspace, Q as it is loaded), so the
    output equals, bit for bit, the fp16 launch on the fp16-rounded inputs:
    a head read from the wrong workspace slot would differ."""
    import torch
    from llmr_amd import ops
    g = torch.Generator(device="cpu").manual_seed(H * 1000 + S)
    q, k, v = (torch.randn(H, S, 128, generator=g) * 2 for _ in range(3))
    if xtype == 30:
        q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    q, k, v = (t.to(dev) for t in (q, k, v))
    o_wide = ops.flash_attention(q, k, v, 1.0 / math.sqrt(128))
    o_16 = ops.flash_attention(q.half(), k.half(), v.half(), 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    assert torch.equal(o_wide, o_16)


def test_fa_constant_values(dev):
    """V constant along the keys -> every output row equals that row of V."""
    from llmr_amd import synth
    H, S = 3, 300
    q = synth.normal(2, 3, H * S * 128).reshape(H, S, 128) * 3
    k = synth.normal(2, 4, H * S * 128).reshape(H, S, 128) * 3
    base = synth.normal(2, 5, H * 128).reshape(H, 1, 128)
    v = np.repeat(base, S, axis=1).astype(np.float16).astype(np.float32)
    o, _ = _fa(dev, q, k, v, 1)
    exp = np.transpose(v, (1, 0, 2)).reshape(S, H * 128)
    assert np.max(np.abs(o - exp)) <= 2e-3 * np.max(np.abs(exp))


def test_fa_key_permutation_invariance(dev):
    from llmr_amd import synth
    H, S = 2, 384
    n = H * S * 128
    q = synth.normal(4, 3, n).reshape(H, S, 128)
    k = synth.normal(4, 4, n).reshape(H, S, 128)
    v = synth.normal(4, 5, n).reshape(H, S, 128)
    perm = np.random.default_rng(0).permutation(S)
    o1, _ = _fa(dev, q, k, v, 1)
    o2, _ = _fa(dev, q, k[:, perm], v[:, perm], 1)
    assert rel_l2(o2, o1) <= 1e-3


def test_fa_flux_full_size_sampled(orc, dev):
    """Flux shape (H=24, S=4608, f16, RoPE applied): the oracle checks sampled
    (head, query-block) pairs; the whole output is checked for finiteness and
    for the convex-combination bound |O| <= max|V| per head and dim."""
    import torch
    from llmr_amd import ops, workloads
    a = workloads.FLUX_ATTENTION
    q, k, v = workloads.attention_inputs(a)
    qt, kt, vt = (torch.from_numpy(t).to(dev) for t in (q, k, v))
    o = ops.flash_attention(qt, kt, vt, 1.0 / math.sqrt(a.D))
    torch.cuda.synchronize()
    o = o.cpu().numpy()
    assert np.all(np.isfinite(o))
    vmax = np.abs(v.astype(np.float32)).max(axis=1)  # [H, D]
    assert np.all(np.abs(o.reshape(a.S, a.H, a.D)) <= vmax[None] * (1 + 1e-3) + 1e-6)
    for h, q0 in [(0, 0), (7, 512), (23, a.S - 128), (12, 2048)]:
        ref = orc.flash_attention(q[h:h + 1].astype(np.float32), k[h:h + 1].astype(np.float32),
                                  v[h:h + 1].astype(np.float32), 1.0 / math.sqrt(a.D),
                                  qrange=(q0, q0 + 128))
        got = o.reshape(a.S, a.H, a.D)[q0:q0 + 128, h]
        err = rel_l2(got, ref.reshape(a.S, a.D)[q0:q0 + 128])
        print(f"head {h} q {q0}: rel_l2={err:.3e}")
        assert err <= TOL


@pytest.mark.parametrize("otype,H,S,pad", [("bfloat16", 2, 300, 40), ("float16", 3, 257, 0), ("float32", 2, 129, 8),
                                           ("bfloat16", 24, 4608, 0)])
def test_fa_rows_equal_f32_output_rounded(dev, otype, H, S, pad):
    """llmr_flash_attention_rows writes the f32 attention rows rounded to the
    output type (nearest even), at a row stride with a column offset, and
    touches nothing else of the destination: bit for bit the f32 launch
    followed by a torch cast (the values llmr_activation's copy gives)."""
    import torch
    from llmr_amd import ops
    dt = getattr(torch, otype)
    g = ops.default_graph()
    gen = torch.Generator(device="cpu").manual_seed(S + H)
    q, k, v = (torch.randn(H, S, 128, generator=gen).half().to(dev) for _ in range(3))
    pc = ops.FlashAttentionPC(128, H, S, 1.0 / 128 ** 0.5)
    ref = torch.empty(S, H * 128, dtype=torch.float32, device=dev)
    ops.dispatch_flash_attention(g, *(ops.Tensor.from_torch(t) for t in (q, k, v)), ops.Tensor.from_torch(ref), pc)
    width = H * 128 + 64 + pad
    dst = torch.full((S, width), 7.0, dtype=dt, device=dev)
    ops.dispatch_flash_attention_rows(g, *(ops.Tensor.from_torch(t) for t in (q, k, v)), dst[:, 64:64 + H * 128], pc)
    torch.cuda.synchronize()
    assert torch.equal(dst[:, 64:64 + H * 128], ref.to(dt))
    assert (dst[:, :64] == 7.0).all() and (dst[:, 64 + H * 128:] == 7.0).all()
