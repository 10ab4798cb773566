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


def _check_plan(groups, cus, wtype=None):
    """Every panel of every image of each group after the first built
    exactly once, by call k - 1, k - 2 or k - 3 (never into the buffer the
    building call reads: group k in buffer k % 4); at most eight parts a
    call; group k + 1's parts first, and the parts of the groups after it
    only within three quarters of what is left of the call's room. Returns
    the plan and the items each call leaves to the image launch after its
    GEMM."""
    C = dit._ImageChain
    kw = {} if wtype is None else {"wtype": wtype}
    builds = C.plan(groups, cus, **kw)
    seen = {}
    left = []
    for c, parts in enumerate(builds):
        assert len(parts) <= C.MAX_PARTS, c
        room = C._room(groups[c], cus, **kw)
        nxt = sum((p1 - p0) * C._stage_groups(groups[j]) for j, e, p0, p1 in parts if j == c + 1)
        later = sum((p1 - p0) * C._stage_groups(groups[j]) for j, e, p0, p1 in parts if j > c + 1)
        assert later <= max(0, room - nxt) * 3 // 4, c
        js = [j for j, _, _, _ in parts]
        assert js == sorted(js) and all(1 <= j - c <= C.NBUF - 1 for j in js), (c, parts)
        for j, e, p0, p1 in parts:
            assert j % C.NBUF != c % C.NBUF and 0 <= p0 < p1 <= C._entry_panels(groups[j])[e], (c, j, e)
            for p in range(p0, p1):
                assert (j, e, p) not in seen, (c, j, e, p)
                seen[(j, e, p)] = c
        left.append(max(0, nxt + later - room))
    want = {(j, e, p) for j in range(1, len(groups)) for e, n in enumerate(C._entry_panels(groups[j]))
            for p in range(n)}
    assert set(seen) == want
    return builds, left


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
    QKV builds the projection's images and, in three quarters of what is
    left of its room, the MLP-in's text image and half its image-row one;
    the projection the rest of that and three panels of the MLP-out's."""
    groups = _flux_groups("gelu")
    builds, left = _check_plan(groups, 256)
    assert sum(left) == 0
    assert builds[0] == [(1, 0, 0, 12), (1, 1, 0, 12), (2, 0, 0, 48), (2, 1, 0, 24)]
    assert builds[1] == [(2, 1, 24, 48), (3, 0, 0, 3)]


def test_image_chain_plan_flux2_step():
    """The Flux.2 form: the MLP-in's images (SwiGLU only) and linear1's
    (plain Q | K | V rows, then the SwiGLU rows: two images of one weight)
    take part, and a call with room left after the next group builds parts
    of the two groups after it (within three quarters of that room): the
    MLP-out begins the next block's MLP-in (42 of its text image's 96
    panels), so from the second double block on 624 items a block are left
    to launches (the first block 1344), against 1056 a block when only the
    next two groups' whole images were planned."""
    C = dit._ImageChain
    groups = _flux_groups("swiglu")
    assert C._entries(groups[2]) == 2 and C._entries(groups[76]) == 2
    # the split SwiGLU weight's panels: 36 plain + 96 of 128 outputs
    assert C._panels(groups[76]) == 132 and C._entry_items(groups[76]) == [36 * 12, 96 * 12]
    builds, left = _check_plan(groups, 256)
    assert left[:8] == [0, 960, 384, 0, 0, 240, 384, 0] and sum(left) == 1344 + 18 * 624
    assert builds[3] == [(4, 0, 0, 36), (4, 1, 0, 36), (5, 0, 0, 12), (5, 1, 0, 12), (6, 0, 0, 42)]
    assert builds[4] == [(6, 0, 42, 96), (6, 1, 0, 36)]


def test_image_chain_plan_zimage_block():
    """The Z-Image block's four Q8_0 GEMMs (QKV, O-proj, SwiGLU, down):
    with one item per eight K stages of room the QKV and the O-proj build
    a few items of the next image each and the SwiGLU (176 idle
    workgroups) the down projection's whole image."""
    from llmr_amd.gguf import GGML_Q8_0
    d, f, S = 3840, 10240, 4352
    groups = [([0], 3 * d, d, (S,)), ([0], d, d, (S,)), ([0], 2 * f, d, (S,), 0), ([0], d, f, (S,))]
    builds, left = _check_plan(groups, 256, GGML_Q8_0)
    assert builds[:3] == [[(1, 0, 0, 15)], [(2, 0, 0, 80)], [(3, 0, 0, 15)]]
    assert left[2] == 0 and left[0] > 0 and left[1] > 0


def test_image_chain_plan_eight_images():
    """A call builds no more than the eight next images a call takes: of four
    split SwiGLU weights' eight images after a group whose room would hold
    them all, the last is left to the next call."""
    groups = [([0, 1], 1024, 1024, (300,)), ([0], 1024, 1024, (256,)), ([0, 1, 2, 3], 2048, 1024, (256,), 512),
              ([0], 1024, 1024, (256,))]
    C = dit._ImageChain
    assert C._entries(groups[2]) == 8
    assert C._items(groups[1]) + C._items(groups[2]) <= C._room(groups[0], 256)
    builds, _ = _check_plan(groups, 256)
    assert len(builds[0]) == 8 and builds[0][0] == (1, 0, 0, 4) and builds[0][-1] == (2, 6, 0, 2)
    assert builds[1][0] == (2, 7, 0, 6)  # f = 768 outputs: six panels


def test_image_chain_plan_random_groups():
    """The planner's rules (_check_plan) over 300 random group sequences:
    one or two weights (up to four for split SwiGLU groups of one
    projection), N and K multiples of 64 of a few hundred to several
    thousand, plain or split SwiGLU groups (split 0 or a multiple of 256),
    one or two jobs of 1-5000 tokens, 80-304 CUs, Q4_K and Q8_0 rooms."""
    import random
    from llmr_amd.gguf import GGML_Q4_K, GGML_Q8_0
    rnd = random.Random(20261202)
    C = dit._ImageChain
    for _ in range(300):
        groups = []
        for _ in range(rnd.randint(2, 14)):
            K = 64 * rnd.randint(1, 120)
            Ms = tuple(rnd.randint(1, 5000) for _ in range(rnd.randint(1, 2)))
            if rnd.random() < 0.3:  # split SwiGLU: split rows plain, then 2 f SwiGLU rows
                split = 256 * rnd.randint(0, 12)
                f = 8 * rnd.randint(1, 600)
                nw = rnd.randint(1, 4 if split == 0 else 2)
                groups.append(([0] * nw, split + 2 * f, K, Ms, split))
            else:
                groups.append(([0] * rnd.randint(1, 2), 64 * rnd.randint(1, 300), K, Ms))
        assert all(C._entries(gr) <= C.MAX_PARTS for gr in groups)
        _check_plan(groups, rnd.choice((80, 104, 256, 304)), rnd.choice((GGML_Q4_K, GGML_Q8_0)))
