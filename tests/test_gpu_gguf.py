"""GGUF checkpoint -> device: tensors uploaded by the native loader feed the
GEMM unchanged, and a whole Flux forward from a checkpoint written with the
BFL tensor names equals the forward from the in-memory weights bit for bit."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def test_uploaded_q4k_weight_feeds_the_gemm(orc, dev, tmp_path):
    import torch
    from llmr_amd import gguf, gguf_file, ops
    r = np.random.default_rng(9)
    N, K, M = 320, 1024, 200
    w = (0.02 * r.standard_normal((N, K))).astype(np.float32)
    blk = gguf_file.encode_tensor(w, gguf.GGML_Q4_K)
    p = str(tmp_path / "w.gguf")
    gguf_file.write_gguf(p, [gguf_file.TensorEntry("lin.weight", gguf.GGML_Q4_K, (N, K), blk)])
    x = torch.randn(M, K, device=dev).bfloat16()
    with gguf_file.GGUFFile(p) as f:
        wd = f.upload("lin.weight", dev)
    direct = torch.from_numpy(np.frombuffer(blk, np.uint8).copy()).to(dev)
    assert torch.equal(wd, direct)
    y = ops.batch_matmul(wd, gguf.GGML_Q4_K, x, N)
    y2 = ops.batch_matmul(direct, gguf.GGML_Q4_K, x, N)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref = orc.batch_matmul(np.frombuffer(blk, np.uint8), gguf.GGML_Q4_K, x.float().cpu().numpy(), N, K, M, 0)
    assert rel_l2(y.cpu().numpy(), ref) < 1e-2


def test_flux_forward_from_checkpoint_is_identical(dev, tmp_path):
    import torch
    from llmr_amd import dit, synth
    cfg = dit.FluxConfig(dim=256, n_heads=2, mlp=512, n_double=2, n_single=2, text_dim=256, n_txt=40,
                         latent_ch=16, latent_h=16, latent_w=16, patch=2)
    weights = dit.flux_weights(cfg, device=dev)
    p = str(tmp_path / "flux.gguf")
    dit.save_flux_gguf(p, cfg, *weights)
    loaded = dit.flux_weights_from_gguf(p, cfg, device=dev)
    lat = torch.from_numpy(synth.normal(42, 601, 16 * 16 * 16).reshape(16, 16, 16)).to(dev)
    txt = torch.from_numpy(synth.normal(42, 602, cfg.n_txt * cfg.text_dim).reshape(cfg.n_txt, -1)).to(dev)
    txt = txt.to(torch.bfloat16)
    a = dit.FluxDiT(cfg, *weights, device=dev).forward(lat, txt, 0.5).clone()
    b = dit.FluxDiT(cfg, *loaded, device=dev).forward(lat, txt, 0.5)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
    with pytest.raises(ValueError):  # a checkpoint of other shapes is refused
        dit.flux_weights_from_gguf(p, dit.FluxConfig(dim=256, n_heads=2, mlp=768, n_double=2, n_single=2,
                                                     text_dim=256, n_txt=40, latent_ch=16, latent_h=16,
                                                     latent_w=16, patch=2), device=dev)
