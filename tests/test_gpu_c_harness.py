"""A plain C11 program (tests/c/zimage_layer.c, gcc against
include/llmr_hip.h, linked to libllmr_hip.so) replays the Z-Image layer the
way the reference's C3 host issues it: f32 activation buffers, every GEMM
through llmr_batch_matmul_pc with a filled-in BatchMatMulPC, the SwiGLU
through llmr_batch_matmul_swiglu_pc and attention through
llmr_flash_attention_pc (dit_transformer_layer, dependencies/zimage.c3l/
dit.c3:1372-1627). Its output is compared with the oracle's restatement of
the layer (oracle/blocks.py) at small, ragged shapes.

Bar: relative L2 <= 1e-2 on the layer's residual update (f32 inputs: the Q8_0
GEMMs round x to fp16 as the reference does; the SwiGLU rounds x to bf16)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import rel_l2
from test_capi_boundary import _c_harness

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim,heads,ffn,seq", [(256, 2, 512, 200), (384, 3, 640, 77)])
def test_c_caller_zimage_layer_vs_oracle(dev, tmp_path, dim, heads, ffn, seq):
    from llmr_amd import gguf, synth, workloads
    from oracle import blocks
    base = 800 + dim
    r = lambda n, s, std=1.0: synth.normal(42, base + s, n, std)  # noqa: E731
    q8 = lambda rows, cols, s: gguf.quantize(r(rows * cols, s, 0.05).reshape(rows, cols), gguf.GGML_Q8_0)  # noqa: E731
    w = dict(wqkv=q8(3 * dim, dim, 1), wo=q8(dim, dim, 2), w_gate=q8(ffn, dim, 3), w_up=q8(ffn, dim, 4),
             w_down=q8(dim, ffn, 5), attn_norm1=1 + r(dim, 6, 0.1), attn_norm2=1 + r(dim, 7, 0.1),
             ffn_norm1=1 + r(dim, 8, 0.1), ffn_norm2=1 + r(dim, 9, 0.1), q_norm=1 + r(128, 10, 0.1),
             k_norm=1 + r(128, 11, 0.1), adaln=r(4 * dim, 12, 0.6).reshape(4, dim))
    hidden = r(seq * dim, 13).reshape(seq, dim)
    att = workloads.Attention("z", heads, seq, 128, 11, 8, 12, (32, 48, 48), 256.0)
    cos_t, sin_t = workloads.rope_tables(workloads.attention_positions(att), att.axes, att.theta)
    files = dict(w, hidden=hidden, rope_cos=cos_t, rope_sin=sin_t)
    for name, a in files.items():
        ext = "q8" if a.dtype == np.uint8 else "f32"
        (tmp_path / f"{name}.{ext}").write_bytes(np.ascontiguousarray(a, a.dtype if ext == "q8" else np.float32)
                                                  .tobytes())
    exe = _c_harness("zimage_layer")
    print(f"C caller: dim={dim} heads={heads} ffn={ffn} seq={seq}", flush=True)
    res = subprocess.run([exe, str(tmp_path), str(dim), str(heads), str(ffn), str(seq)], capture_output=True,
                         text=True, timeout=60)
    print(res.stdout, res.stderr)
    assert res.returncode == 0, res.stderr
    assert "slots_equal=1" in res.stdout
    got = np.fromfile(tmp_path / "out.f32", np.float32).reshape(seq, dim)
    ref = blocks.zimage_layer(w, hidden, heads, cos_t, sin_t)
    err = rel_l2(got - hidden, ref - hidden)
    print(f"C caller zimage layer: update rel L2 {err:.2e}")
    assert np.isfinite(got).all()
    assert err < 1e-2
