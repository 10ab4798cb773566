"""Host logic of the composed Flux forward (no GPU compute): the weight-image
chain hands each GEMM group the images built for it, matched by position,
which the C-ABI cannot check, so the chain refuses a call whose weights are
not the group's and a failed forward leaves no half-taken chain behind."""
import pytest
import torch

from llmr_amd import dit, gguf, ops


def _q4(rows, K):
    return ops.Tensor.quantized(torch.zeros(rows * gguf.row_bytes(gguf.GGML_Q4_K, K), dtype=torch.uint8),
                                gguf.GGML_Q4_K, rows, K)


def test_image_chain_refuses_out_of_step_calls():
    a, b, c = _q4(256, 256), _q4(256, 256), _q4(512, 256)
    chain = dit._ImageChain([([a, b], 256, 256), ([c], 512, 256)], gguf.GGML_BF16, "cpu")
    chain.k, chain.active = 0, True
    x = ops.Tensor.from_torch(torch.zeros(4, 256, dtype=torch.bfloat16))
    job = lambda w: ops.MatmulJob(w, x, torch.zeros(4, w.shape[0]), 4)  # noqa: E731
    # the group's own weights in order: its images, the next group's to build
    images, nxt = chain.take([job(a), job(b)], 256, 256)
    assert len(images) == 2 and nxt is not None and chain.active
    # a call with other weights than group 1's is refused and ends the chain
    with pytest.raises(RuntimeError, match="out of step"):
        chain.take([job(a)], 512, 256)
    assert not chain.active
