"""One Z-Image DiT block at its full size (hidden 3840, 30 heads x 128,
SwiGLU FFN 10240, 4096 image + 256 text tokens, Q8_0 weights ~N(0, 0.02),
bf16 GEMM inputs; dit_transformer_layer, dependencies/zimage.c3l/
dit.c3:1372-1627) against the oracle's restatement of the layer
(oracle/blocks.py zimage_layer) on sampled rows: the oracle computes K and V
of every token and the rest of the layer on those rows.

The bar is relative L2 <= 1e-2 on what the block adds to the residual
stream (bf16 GEMM inputs and fp16 Q/K/V on the device; the reference's fp16
GEMM operands and f32 elsewhere in the oracle)."""
import numpy as np
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu

# rows across the sequence: the first, one past the first 256, interior, the last
ROWS = np.array([0, 1, 255, 256, 1031, 2600, 4095, 4351])


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def test_zimage_block_full_size_vs_oracle(dev):
    from llmr_amd import dit, synth, workloads
    from oracle import blocks
    dim, H, ffn = 3840, 30, 10240
    a = workloads.ZIMAGE_ATTENTION
    S = a.S
    assert (S, a.H) == (4352, H)
    w = dit.zimage_layer_weights(dim, H, ffn, device=dev, base_stream=900)
    cos_t, sin_t = workloads.rope_tables(workloads.attention_positions(a), a.axes, a.theta)
    h0 = workloads.round_bf16(synth.normal(42, 901, S * dim).reshape(S, dim))
    blk = dit.ZImageBlock(dim, H, ffn, S, act_dtype=torch.bfloat16, device=dev)
    h = torch.from_numpy(h0.copy()).to(dev)
    print(f"zimage block full size: S={S} dim={dim} heads={H} ffn={ffn} rows={ROWS.tolist()}", flush=True)
    blk.forward(w, h, torch.from_numpy(cos_t).to(dev), torch.from_numpy(sin_t).to(dev))
    torch.cuda.synchronize()
    got = _np(h)
    assert np.isfinite(got).all()
    wn = {k: _np(getattr(w, k)) for k in w.__dataclass_fields__}
    ref = blocks.zimage_layer(wn, h0, H, cos_t, sin_t, rows=ROWS)
    err = rel_l2(got[ROWS] - h0[ROWS], ref - h0[ROWS])
    print(f"zimage block full size: update rel L2 {err:.2e} on rows {ROWS.tolist()}")
    assert err < 1e-2
