"""GPU: page reset and state copy kernels execute the host plans
(host.page_spans, ResidentPages.copy_plan; native/src/page_binding.h:19-35,161-187)
bit-exactly against numpy; misaligned spans, out-of-field spans and HIP-graph
replays with new plans."""
import numpy as np
import pytest

from ironpangu_amd.host import ResidentPages, page_spans

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_copy_plan_between_residents():
    import torch
    from ironpangu_amd import ops
    page_tokens, logical, slots = 32, 1024, 4
    pages = ResidentPages(page_tokens, logical, slots, shared=True)
    rng = np.random.default_rng(0)
    perm = rng.permutation(logical // page_tokens * slots).astype(np.int32)
    for slot in range(slots):
        pages.release(slot)
    pages.select(0)
    pages.bind(perm[:32])
    pages.select(1)
    pages.bind(perm[32:64])
    page_bytes = page_tokens * 656
    field_bytes = 128 * page_bytes
    field = rng.integers(0, 256, field_bytes, dtype=np.uint8)
    plan = pages.copy_plan(0, 1, 512, False, field_bytes)
    exp = field.copy()
    for s, d, b in plan:
        exp[d:d + b] = field[s:s + b]
    t = dev(field)
    ops.state_copy(t, dev(np.array(plan, np.uint64).view(np.int64)))
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), exp)


@pytest.mark.parametrize("page_bytes", [20992, 20])  # 16-byte aligned pages and a byte path
def test_page_reset_spans(page_bytes):
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(1)
    n_pages = 200
    field = rng.integers(1, 256, n_pages * page_bytes, dtype=np.uint8)
    owned = rng.choice(n_pages, 57, replace=False).astype(np.int32)
    spans = page_spans(owned, page_bytes, field.size)
    exp = field.copy()
    for o, b in spans:
        exp[o:o + b] = 0
    plan = np.array(spans + [(field.size - 8, 64)], np.uint64)  # last span leaves the field: skipped
    t = dev(field)
    ops.page_reset(t, dev(plan.view(np.int64)))
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), exp)


def test_graph_replay_reads_new_plans():
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(2)
    page_bytes, n_pages = 4096, 64
    base = rng.integers(0, 256, n_pages * page_bytes, dtype=np.uint8)
    t = dev(base)
    plan = torch.zeros((4, 3), dtype=torch.int64, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        ops.state_copy(t, plan, stream=s)  # warm-up outside capture (zero-byte ranges)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            ops.state_copy(t, plan, stream=s)
    for rep in range(3):
        srcs = rng.choice(32, 4, replace=False)
        dsts = 32 + rng.choice(32, 4, replace=False)
        p = np.stack([srcs * page_bytes, dsts * page_bytes, np.full(4, page_bytes)], 1)
        cur = t.cpu().numpy()
        exp = cur.copy()
        for a, b, n in p:
            exp[b:b + n] = cur[a:a + n]
        plan.copy_(dev(p.astype(np.int64)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(t.cpu().numpy(), exp), rep


def test_overlapping_copy_range_is_skipped():
    """A range whose source and destination overlap is skipped; the other
    ranges of the same plan are copied."""
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(3)
    field = rng.integers(0, 256, 1 << 16, dtype=np.uint8)
    plan = np.array([[0, 4096, 8192], [32768, 49152, 4096]], np.uint64)  # first overlaps itself
    exp = field.copy()
    exp[49152:53248] = field[32768:36864]
    t = dev(field)
    ops.state_copy(t, dev(plan.view(np.int64)))
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), exp)


@pytest.mark.parametrize("bad", ["overlap", "outside", "empty", "none"])
def test_checked_copy_is_all_or_nothing(bad):
    """The checked entry point validates the whole plan with the reference's rule
    (prepared_execution.h:346-354): one bad range and no byte moves, the status
    names it (1-based); a valid plan copies as the unchecked call."""
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(4)
    field = rng.integers(0, 256, 1 << 16, dtype=np.uint8)
    plan = [[0, 16384, 4096], [32768, 49152, 4096], [4096, 20480, 4096]]
    third = {"overlap": [8192, 9216, 4096], "outside": [60000, 4096, 8192],
             "empty": [0, 4096, 0], "none": [12288, 28672, 4096]}[bad]
    plan.insert(2, third)
    t = dev(field)
    status = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    ops.state_copy(t, dev(np.array(plan, np.int64)), status=status)
    torch.cuda.synchronize()
    got = t.cpu().numpy()
    if bad == "none":
        exp = field.copy()
        for s, d, n in plan:
            exp[d:d + n] = field[s:s + n]
        assert status.item() == 0
        assert np.array_equal(got, exp)
    else:
        assert status.item() == 3
        assert np.array_equal(got, field)


def test_checked_reset_is_all_or_nothing():
    import torch
    from ironpangu_amd import ops
    field = np.full(1 << 14, 9, np.uint8)
    t = dev(field)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.page_reset(t, dev(np.array([[0, 4096], [16000, 4096]], np.int64)), status=status)
    torch.cuda.synchronize()
    assert status.item() == 2 and np.array_equal(t.cpu().numpy(), field)
    ops.page_reset(t, dev(np.array([[0, 4096], [8192, 4096]], np.int64)), status=status)
    torch.cuda.synchronize()
    exp = field.copy()
    exp[0:4096] = 0
    exp[8192:12288] = 0
    assert status.item() == 0 and np.array_equal(t.cpu().numpy(), exp)
