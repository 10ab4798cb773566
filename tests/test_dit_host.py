"""Host logic of the composed Flux forward (no GPU compute): the weight-image
chain hands each GEMM group the images built for it, matched by position,
which the C-ABI cannot check, so the chain refuses a call whose weights are
not the group's and a failed forward leaves no half-taken chain behind; its
plan has each group's images built once, by one of the two calls before it,
into a buffer no call between reads."""
import pytest
import torch

from llmr_amd import dit, gguf, ops


def _q4(rows, K):
    return ops.Tensor.quantized(torch.zeros(rows * gguf.row_bytes(gguf.GGML_Q4_K, K), dtype=torch.uint8),
                                gguf.GGML_Q4_K, rows, K)


def test_image_chain_refuses_out_of_step_calls():
    a, b, c = _q4(256, 256), _q4(256, 256), _q4(512, 256)
    chain = dit._ImageChain([([a, b], 256, 256, (256, 256)), ([c], 512, 256, (512,))], gguf.GGML_BF16, "cpu", 256)
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


def test_image_chain_plan_flux_step():
    """The plan over a Flux-dev step's GEMM groups (19 double blocks: QKV,
    projection, MLP-in, MLP-out of the text and image rows; 38 single
    blocks: linear1, linear2) on 256 CUs: each group after the first is
    built by call k - 1 or k - 2 and by no other, never into the buffer the
    building call reads (k % 3), and within the room of every call that
    builds two groups. Where the rooms allow it (the double block's QKV
    builds the projection's and the MLP-in's images, linear2 the next
    linear1's and linear2's) no call is left with a group it cannot build
    on its idle workgroups."""
    d, m, S, nt = 3072, 12288, 4608, 512
    two = (nt, S - nt)
    groups = []
    for _ in range(19):
        groups += [([0, 1], 3 * d, d, two), ([0, 1], d, d, two), ([0, 1], m, d, two), ([0, 1], d, m, two)]
    for _ in range(38):
        groups += [([0], 3 * d + m, d, (S,)), ([0], d, d + m, (S,))]
    builds = dit._ImageChain.plan(groups, 256)
    by = {}
    for c, js in enumerate(builds):
        for j in js:
            assert j not in by and j - c in (1, 2) and j % 3 != c % 3, (c, j)
            by[j] = c
        if len(js) == 2:
            assert sum(dit._ImageChain._items(groups[j]) for j in js) <= dit._ImageChain._room(groups[c], 256), c
    assert sorted(by) == list(range(1, len(groups)))
    # no group is left to a call whose room cannot hold it
    for j, c in by.items():
        if j == c + 1 and len(builds[c]) == 1:
            assert dit._ImageChain._items(groups[j]) <= dit._ImageChain._room(groups[c], 256), (c, j)
    assert builds[0] == [1, 2] and builds[1] == [] and builds[2] == [3] and builds[3] == [4, 5]
    s0 = 19 * 4
    assert builds[s0] == [] and builds[s0 + 1] == [s0 + 2, s0 + 3]
