"""The Flux-dev-shaped DiT at full size (hidden 3072, 24 heads, MLP 12288,
512 text + 4096 image tokens, Q4_K weights): one double block and one
single block against the oracle's block restatement (oracle/blocks.py) on
sampled rows, and the whole 19 + 38 block denoising step for finite,
deterministic output.

The bar is relative L2 <= 1e-2 on what a block adds to the residual stream
(bf16 GEMM inputs, fp16 Q/K/V on the device; f32 throughout in the oracle)."""
import numpy as np
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu

# joint rows checked: text rows (first, middle, last) and image rows
# (first, interior, last); the oracle computes K/V for every row
ROWS = np.array([0, 1, 255, 511, 512, 513, 2600, 4607])


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def _as_np(o):
    return {k: _np(getattr(o, k)) for k in o.__dataclass_fields__}


@pytest.fixture(scope="module")
def flux1(dev):
    """A full-shape model with one double and one single block, its stream
    filled with N(0, 1) and its modulation vectors with N(0, 0.5^2)."""
    from llmr_amd import dit, synth
    cfg = dit.FluxConfig(n_double=1, n_single=1)
    glob, doubles, singles = dit.flux_weights(cfg, device=dev)
    model = dit.FluxDiT(cfg, glob, doubles, singles, device=dev)
    h0 = synth.normal(42, 710, cfg.seq * cfg.dim).reshape(cfg.seq, cfg.dim)
    mods = synth.normal(42, 711, model.mods.numel(), 0.5).reshape(1, -1)
    model.mods.copy_(torch.from_numpy(mods))
    cos_t, sin_t = (_np(t) for t in model.rope)
    return cfg, model, doubles[0], singles[0], h0, cos_t, sin_t


def test_flux_double_block_full_shape_vs_oracle(flux1):
    from oracle import blocks
    cfg, model, w, _, h0, cos_t, sin_t = flux1
    nt = cfg.n_txt
    model.hidden.copy_(torch.from_numpy(h0))
    mi, mt = model._mod(0, 6), model._mod(6, 6)
    print(f"double block: S={cfg.seq} dim={cfg.dim} rows={ROWS.tolist()}", flush=True)
    model._double(w, mi, mt)
    torch.cuda.synchronize()
    got = _np(model.hidden)[ROWS]
    ref = blocks.flux_double_block(_as_np(w), h0[:nt], h0[nt:], _np(mt), _np(mi), cfg.n_heads, cos_t, sin_t,
                                   rows=ROWS)
    assert np.isfinite(got).all()
    for name, sel in (("text", ROWS < nt), ("image", ROWS >= nt)):
        err = rel_l2(got[sel] - h0[ROWS[sel]], ref[sel] - h0[ROWS[sel]])
        print(f"double block {name} rows: update rel L2 {err:.2e}")
        assert err < 1e-2


def test_flux_single_block_full_shape_vs_oracle(flux1):
    from oracle import blocks
    cfg, model, _, w, h0, cos_t, sin_t = flux1
    model.hidden.copy_(torch.from_numpy(h0))
    ms = model._mod(12, 3)
    print(f"single block: S={cfg.seq} dim={cfg.dim} rows={ROWS.tolist()}", flush=True)
    model._single(w, ms)
    torch.cuda.synchronize()
    got = _np(model.hidden)[ROWS]
    ref = blocks.flux_single_block(_as_np(w), h0, _np(ms), cfg.n_heads, cos_t, sin_t, rows=ROWS)
    assert np.isfinite(got).all()
    err = rel_l2(got - h0[ROWS], ref - h0[ROWS])
    print(f"single block: update rel L2 {err:.2e}")
    assert err < 1e-2


@pytest.fixture(scope="module")
def flux2(dev):
    """The same at full shape with the reference's own Flux.2 MLP form:
    linear1 [3 dim + 2 mlp, dim] and MLP in-projections [2 mlp, dim] whose
    gate and up halves the GEMMs' split-SwiGLU epilogue combines."""
    from llmr_amd import dit, synth
    cfg = dit.FluxConfig(n_double=1, n_single=1, mlp_act="swiglu")
    glob, doubles, singles = dit.flux_weights(cfg, device=dev)
    model = dit.FluxDiT(cfg, glob, doubles, singles, device=dev)
    h0 = synth.normal(42, 720, cfg.seq * cfg.dim).reshape(cfg.seq, cfg.dim)
    mods = synth.normal(42, 721, model.mods.numel(), 0.5).reshape(1, -1)
    model.mods.copy_(torch.from_numpy(mods))
    cos_t, sin_t = (_np(t) for t in model.rope)
    return cfg, model, doubles[0], singles[0], h0, cos_t, sin_t


def test_flux2_double_block_full_shape_vs_oracle(flux2):
    from oracle import blocks
    cfg, model, w, _, h0, cos_t, sin_t = flux2
    nt = cfg.n_txt
    model.hidden.copy_(torch.from_numpy(h0))
    mi, mt = model._mod(0, 6), model._mod(6, 6)
    print(f"Flux.2 double block: S={cfg.seq} dim={cfg.dim} rows={ROWS.tolist()}", flush=True)
    model._double(w, mi, mt)
    torch.cuda.synchronize()
    got = _np(model.hidden)[ROWS]
    ref = blocks.flux_double_block(_as_np(w), h0[:nt], h0[nt:], _np(mt), _np(mi), cfg.n_heads, cos_t, sin_t,
                                   rows=ROWS, mlp_act="swiglu")
    assert np.isfinite(got).all()
    for name, sel in (("text", ROWS < nt), ("image", ROWS >= nt)):
        err = rel_l2(got[sel] - h0[ROWS[sel]], ref[sel] - h0[ROWS[sel]])
        print(f"Flux.2 double block {name} rows: update rel L2 {err:.2e}")
        assert err < 1e-2


def test_flux2_single_block_full_shape_vs_oracle(flux2):
    from oracle import blocks
    cfg, model, _, w, h0, cos_t, sin_t = flux2
    model.hidden.copy_(torch.from_numpy(h0))
    ms = model._mod(12, 3)
    print(f"Flux.2 single block: S={cfg.seq} dim={cfg.dim} rows={ROWS.tolist()}", flush=True)
    model._single(w, ms)
    torch.cuda.synchronize()
    got = _np(model.hidden)[ROWS]
    ref = blocks.flux_single_block(_as_np(w), h0, _np(ms), cfg.n_heads, cos_t, sin_t, rows=ROWS, mlp_act="swiglu")
    assert np.isfinite(got).all()
    err = rel_l2(got - h0[ROWS], ref - h0[ROWS])
    print(f"Flux.2 single block: update rel L2 {err:.2e}")
    assert err < 1e-2


def test_flux_dev_step_full_size_finite_and_deterministic(dev):
    """The whole 19 + 38 block step (the bench's flux_step) twice on the same
    inputs: finite, bit-identical, and not degenerate."""
    from llmr_amd import dit, synth
    cfg = dit.FLUX_DEV
    print(f"flux-dev step: {cfg.n_double}+{cfg.n_single} blocks, S={cfg.seq}", flush=True)
    model = dit.FluxDiT(cfg, *dit.flux_weights(cfg, device=dev), device=dev)
    lat = torch.from_numpy(synth.normal(42, 30, cfg.latent_ch * cfg.latent_h * cfg.latent_w)
                           .reshape(cfg.latent_ch, cfg.latent_h, cfg.latent_w)).to(dev)
    txt = torch.from_numpy(synth.normal(42, 31, cfg.n_txt * cfg.text_dim).reshape(cfg.n_txt, cfg.text_dim))
    txt = txt.to(dev).to(torch.bfloat16)
    a = model.forward(lat, txt, 0.5).clone()
    b = model.forward(lat, txt, 0.5)
    torch.cuda.synchronize()
    assert a.shape == (cfg.latent_ch, cfg.latent_h, cfg.latent_w)
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
    std = float(a.std())
    print(f"velocity std {std:.3e}, max |v| {float(a.abs().max()):.3e}")
    assert std > 1e-3
    del model
    torch.cuda.empty_cache()
