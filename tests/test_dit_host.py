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


def _check_plan(groups, cus):
    """Each image of each group after the first built by call k - 1 or
    k - 2 and by no other, never into the buffer the building call reads
    (k % 3); at most four images a call; a call builds group k + 2's images
    only after all of group k + 1's, and only within its room. Returns the
    plan, (group, image) -> call, and the items a call leaves to the image
    launch after its GEMM."""
    C = dit._ImageChain
    builds = C.plan(groups, cus)
    by = {}
    for c, es in enumerate(builds):
        assert len(es) <= 4, c
        assert es == sorted(es), c
        for j, e in es:
            assert (j, e) not in by and j - c in (1, 2) and j % 3 != c % 3, (c, j, e)
            by[(j, e)] = c
        if any(j == c + 2 for j, _ in es):
            assert sum(C._entry_items(groups[j])[e] for j, e in es) <= C._room(groups[c], cus), c
    assert sorted(by) == [(j, e) for j in range(1, len(groups)) for e in range(C._entries(groups[j]))]
    left = [max(0, sum(C._entry_items(groups[j])[e] for j, e in es) - C._room(groups[c], cus))
            for c, es in enumerate(builds)]
    return builds, by, left


def _flux_groups(act):
    """A Flux-dev step's GEMM groups (19 double blocks: QKV, projection,
    MLP-in, MLP-out of the text and image rows; 38 single blocks: linear1,
    linear2); swiglu: the Flux.2 form, whose MLP-in and linear1 are split
    SwiGLU groups (split 0 and 3 dim)."""
    d, m, S, nt = 3072, 12288, 4608, 512
    two = (nt, S - nt)
    mi, sp0, sp1 = (2 * m, (0,), (3 * d,)) if act == "swiglu" else (m, (), ())
    groups = []
    for _ in range(19):
        groups += [([0, 1], 3 * d, d, two), ([0, 1], d, d, two), ([0, 1], mi, d, two) + sp0, ([0, 1], d, m, two)]
    for _ in range(38):
        groups += [([0], 3 * d + mi, d, (S,)) + sp1, ([0], d, d + m, (S,))]
    return groups


def test_image_chain_plan_flux_step():
    """The plan over a Flux-dev step's GEMM groups on 256 CUs keeps the
    chain's rules and leaves no item to an image launch: the double block's
    QKV builds the projection's and the MLP-in's images, the MLP-in the
    MLP-out's and the next QKV's text image, linear2 the next linear1's and
    linear2's."""
    groups = _flux_groups("gelu")
    builds, _, left = _check_plan(groups, 256)
    assert sum(left) == 0
    assert builds[0] == [(1, 0), (1, 1), (2, 0), (2, 1)] and builds[1] == []
    assert builds[2] == [(3, 0), (3, 1), (4, 0)] and builds[3] == [(4, 1), (5, 0), (5, 1)]
    s0 = 19 * 4
    assert builds[s0] == [] and builds[s0 + 1] == [(s0 + 2, 0), (s0 + 3, 0)]


def test_image_chain_plan_flux2_step():
    """The Flux.2 form: the MLP-in's images (SwiGLU only) and linear1's
    (plain Q | K | V rows, then the SwiGLU rows: two images of one weight)
    take part. The double block's MLP-in is twice as wide, so the QKV no
    longer builds it beside the projection; linear2 still builds the next
    linear1 and linear2 (three images)."""
    C = dit._ImageChain
    groups = _flux_groups("swiglu")
    assert C._entries(groups[2]) == 2 and C._entries(groups[76]) == 2
    # the split SwiGLU weight's panels: 36 plain + 96 of 128 outputs
    assert C._panels(groups[76]) == 132 and C._entry_items(groups[76]) == [36 * 12, 96 * 12]
    builds, _, left = _check_plan(groups, 256)
    # the QKV builds the MLP-in's text image beside the projection's; the
    # projection (room 480) and the MLP-in (room 768) leave 672 and 384
    # items a double block to image launches, the single blocks none
    assert builds[0] == [(1, 0), (1, 1), (2, 0)] and builds[1] == [(2, 1)] and builds[2] == [(3, 0), (3, 1)]
    assert left[:4] == [0, 672, 384, 0] and sum(left) == 19 * (672 + 384)
    s0 = 19 * 4
    assert builds[s0] == [(s0 + 1, 0), (s0 + 2, 0)] and builds[s0 + 1] == [(s0 + 2, 1), (s0 + 3, 0)]


def test_image_chain_plan_four_images():
    """A call builds no more than the four images a call takes: of two split
    SwiGLU weights' four images after a group whose room would hold them
    all, the last is left to the next call."""
    groups = [([0, 1], 1024, 1024, (300,)), ([0], 1024, 1024, (256,)), ([0, 1], 2048, 1024, (256,), 512),
              ([0], 1024, 1024, (256,))]
    C = dit._ImageChain
    assert C._entries(groups[2]) == 4
    assert C._items(groups[1]) + C._items(groups[2]) <= C._room(groups[0], 256)
    builds, _, _ = _check_plan(groups, 256)
    assert builds[0] == [(1, 0), (2, 0), (2, 1), (2, 2)] and builds[1] == [(2, 3), (3, 0)]
