"""Host metadata (slot mapping, block tables, packed varlen layout, page spans,
state copy plans) against (1) the known answers of the reference's own C++
tests, restated here, and (2) vectors produced by the reference's headers
compiled in place (tests/golden/host_meta.json, made by
tests/golden/make_golden.py from oracle/_ref)."""
import json
from pathlib import Path

import numpy as np
import pytest

from ironpangu_amd.host import MetadataError, ResidentPages, SequenceBatch, page_spans

GOLDEN = json.loads((Path(__file__).parent / "golden" / "host_meta.json").read_text())


def rejects(f):
    with pytest.raises(MetadataError):
        f()


# ---- native/probes/page_binding_test.cpp ------------------------------------

@pytest.mark.parametrize("page", [16, 32])
def test_fixed_binding_fragmented_and_rollback(page):
    # PageBinding(page, 3*page, 7).bind({6,0,4}) expressed through a 1-resident
    # table over a 7-page pool is not constructible here (pool = pages per slot
    # x slots), so use the ResidentPages form of the same test (:29-42).
    p = ResidentPages(page, page * 3, 2)
    p.bind([2, 0, 1])
    p.select(1)
    assert p.append(0) == 3 * page
    p.bind([5, 3, 4])
    rejects(lambda: p.bind([0, 3, 4]))          # crosses resident partition
    rejects(lambda: p.select(2))
    assert p.append(0) == 5 * page
    p.select(0)
    assert p.append(0) == 2 * page
    assert p.append(page - 1) == 3 * page - 1
    assert p.append(page) == 0
    assert p.append(3 * page - 1) == 2 * page - 1
    rejects(lambda: p.append(3 * page))
    rejects(lambda: p.bind([3, 0, 1]))
    rejects(lambda: p.bind([0, 0, 1]))          # alias
    rejects(lambda: p.bind([0, -1, 1]))
    rejects(lambda: p.bind([0, 1]))             # length
    assert p.append(0) == 2 * page              # failed update keeps the old map


def test_invalid_capacities():
    rejects(lambda: ResidentPages(0, 32, 2))
    rejects(lambda: ResidentPages(16, 31, 2))
    rejects(lambda: ResidentPages(16, 64, 0))
    rejects(lambda: ResidentPages(16, 64, 65))


@pytest.mark.parametrize("page", [16, 32])
def test_shared_reservations(page):
    # page_binding_test.cpp:44-64
    p = ResidentPages(page, page * 3, 2, shared=True)
    p.release(0)
    p.release(1)
    rejects(lambda: p.append(0))
    p.bind([5, 0])
    assert p.append(0) == 5 * page
    assert p.append(page) == 0
    rejects(lambda: p.append(2 * page))
    p.select(1)
    p.bind([4])
    rejects(lambda: p.bind([5]))
    assert p.append(0) == 4 * page
    p.select(0)
    rejects(lambda: p.bind([1, 4]))  # no partial release/claim on failure
    assert p.append(0) == 5 * page
    rejects(lambda: p.bind([1, 1]))
    rejects(lambda: p.bind([6]))
    rejects(lambda: p.bind([]))
    p.release(0)
    p.select(1)
    p.bind([5, 0, 4])
    assert p.append(2 * page) == 4 * page
    p.release(1)
    rejects(lambda: p.append(0))


# ---- native/probes/sequence_batch_test.cpp ----------------------------------

def test_sequence_batch_mixed_rows():
    b = SequenceBatch.make([(3, 100, 1, True), (0, 4096, 4096, False), (2, 7, 3, True)], 4, 4100, 8192)
    assert b.starts == [0, 1, 4097, 4100]
    assert b.residents == [3, 0, 2]
    assert b.query_ends == [1, 4097, 4100]
    assert b.prior_lengths == [100, 4096, 7]
    assert b.kv_lengths == [101, 8192, 10]
    assert b.sample_rows == [0, 4099]
    assert b.sample_residents == [3, 2]
    for i in range(len(b.positions)):
        slot = 3 if i == 0 else (0 if i < 4097 else 2)
        pos = 100 if i == 0 else (4096 + i - 1 if i < 4097 else 7 + i - 4097)
        assert b.row_residents[i] == slot and b.positions[i] == pos and b.lengths[i] == pos + 1
    for bad in ([], [(0, 0, 1, 1), (0, 1, 1, 1)], [(4, 0, 1, 1)], [(0, 0, 0, 1)],
                [(0, 8192, 1, 1)], [(0, 0xFFFFFFFF, 2, 1)], [(0, 0, 4096, 0), (1, 0, 1, 1)]):
        rejects(lambda: SequenceBatch.make(bad, 4, 4096, 8192))
    rejects(lambda: SequenceBatch.make([(0, 0, 1, 1)], 4, 0xFFFFFFFF, 8192))
    for shared in (False, True):
        pages = ResidentPages(16, 8192, 4, shared)
        pages.select(1)
        selected = pages.append(0)
        slots = pages.slot_mapping(b.row_residents, b.positions)
        assert np.array_equal(slots, np.array(b.row_residents, np.int64) * 8192 + np.array(b.positions))
        assert pages.append(0) == selected  # batch lookups leave the selection alone
        t = pages.batch_table(b.residents, 512, False).reshape(3, 512)
        assert np.array_equal(t, np.array(b.residents)[:, None] * 512 + np.arange(512)[None, :])
        r = pages.batch_table(b.residents, 1025, True).reshape(3, 1025)
        assert np.array_equal(r, np.array(b.residents)[:, None] * 512 + (np.arange(1025) % 512)[None, :])
        rejects(lambda: pages.batch_table([0, 0], 512, False))
        rejects(lambda: pages.batch_table([-1], 512, False))
        rejects(lambda: pages.batch_table([0], 511, False))
        rejects(lambda: pages.append(4, 0))
        if shared:
            pages.release(2)
            rejects(lambda: pages.append(2, 7))
            assert pages.append(0) == selected


@pytest.mark.parametrize("count", [1, 2, 17, 4096])
@pytest.mark.parametrize("position", [0, 511, 4096])
def test_single_sequence_lowering(count, position):
    s = SequenceBatch.make([(0, position, count, False)], 1, 4096, 8192)
    assert s.positions == list(range(position, position + count))
    assert s.lengths == list(range(position + 1, position + count + 1))
    assert s.starts == [0, count]


# ---- native/probes/page_span_test.cpp ----------------------------------------

def _apply_spans(pages, page_bytes, total_pages):
    exp = np.full(total_pages * page_bytes, 0xA7, np.uint8)
    act = exp.copy()
    for p in pages:
        exp[p * page_bytes:(p + 1) * page_bytes] = 0
    n = 0
    for off, size in page_spans(pages, page_bytes, act.size):
        assert off + size <= act.size
        act[off:off + size] = 0
        n += size
    assert np.array_equal(act, exp) and n == len(pages) * page_bytes


@pytest.mark.parametrize("page_bytes", [2, 128, 656, 1152])
def test_page_spans(page_bytes):
    for pages in ([], [4, 0, 3, 1, 8], [0, 2, 4, 6, 8], [9]):
        _apply_spans(pages, page_bytes, 10)


def test_page_spans_64k_coalesce_and_rejects():
    pages = list(range(4095, 2047, -1))
    s = page_spans(pages, 32 * 656, 6144 * 32 * 656)
    assert s == [(2048 * 32 * 656, 2048 * 32 * 656)]
    for args in (([-1], 16, 160), ([10], 16, 160), ([1, 1], 16, 160), ([1], 0, 160),
                 ([1], 16, 159), ([], 16, 0)):
        rejects(lambda: page_spans(*args))


# ---- native/probes/state_copy_plan_test.cpp -----------------------------------

def test_copy_plan_merge_and_rejects():
    p = ResidentPages(32, 128, 3, shared=True)
    assert p.copy_plan(0, 1, 128, False, 384) == [(0, 128, 128)]
    for args in ((0, 0, 64, False, 384), (0, 3, 64, False, 384), (0, 1, 0, False, 384),
                 (0, 1, 63, False, 384), (0, 1, 160, False, 384), (0, 1, 64, False, 383)):
        rejects(lambda: p.copy_plan(*args))
    p.release(1)
    p.select(1)
    p.bind([4])
    rejects(lambda: p.copy_plan(0, 1, 64, False, 384))
    assert p.pages(0) == [0, 1, 2, 3] and p.pages(1) == [4]


@pytest.mark.parametrize("page,capacity,row_bytes,ring", [(16, 544, 1152, True), (32, 4096, 656, False),
                                                           (64, 4096, 128, False)])
@pytest.mark.parametrize("boundary", [64, 512, 576, 4096])
def test_copy_plan_round_trip(page, capacity, row_bytes, ring, boundary):
    # state_copy_plan_test.cpp:14-47 at smaller capacities
    if not ring and boundary > capacity:
        return
    count = capacity // page
    b = ResidentPages(page, capacity, 3, shared=True)
    for s in range(3):
        b.release(s)
    src = [3 * i + 2 for i in range(count)]
    dst = [3 * (count - 1 - i) for i in range(count)]
    b.bind(src)
    b.select(1)
    b.bind(dst)
    b.select(0)
    storage = np.full(capacity * 3 * row_bytes, 0xAB, np.uint8)
    cols = np.arange(row_bytes)
    for tok in range(boundary):
        off = b.append(tok % capacity if ring else tok) * row_bytes
        storage[off:off + row_bytes] = (tok * 17 + cols * 31) % 251
    before = storage.copy()
    total = 0
    for s, d, n in b.copy_plan(0, 1, boundary, ring, storage.size):
        storage[d:d + n] = storage[s:s + n].copy()
        total += n
    assert total == min(capacity, boundary) * row_bytes
    b.select(1)
    first = boundary - capacity if boundary > capacity else 0
    for tok in range(first, boundary):
        off = b.append(tok % capacity if ring else tok) * row_bytes
        assert np.array_equal(storage[off:off + row_bytes], (tok * 17 + cols * 31) % 251)
    for phys in src:
        lo, hi = phys * page * row_bytes, (phys + 1) * page * row_bytes
        assert np.array_equal(before[lo:hi], storage[lo:hi])


# ---- vectors from the reference headers compiled in place ----------------------

def _replay(case):
    p = ResidentPages(case["page"], case["logical"], case["slots"], case["kind"] == "shared")
    for op, arg, status in case["ops"]:
        fn = {"select": p.select, "bind": p.bind, "release": p.release}[op]
        if status == 0:
            fn(arg)
        else:
            rejects(lambda: fn(arg))
    return p


def _or_none(f):
    try:
        return f()
    except MetadataError:
        return None


def test_golden_page_tables():
    for case in GOLDEN["pages"]:
        p = _replay(case)
        got = [_or_none(lambda: p.append(s, q)) for s, q in case["rows"]]
        assert got == case["appends"]
        per = case["logical"] // case["page"]
        if case["kind"] == "fixed":
            assert p.batch_table(case["residents"], per, False).tolist() == case["table"]
            assert p.batch_table(case["residents"], 2 * per + 1, True).tolist() == case["ring"]
        else:
            got_t = _or_none(lambda: p.batch_table(list(range(case["slots"])), per, False).tolist())
            assert got_t == case["table"]
            for a, b, c, w, f, exp in case["copy"]:
                got_c = _or_none(lambda: [list(r) for r in p.copy_plan(a, b, c, w, f)])
                assert got_c == exp


def test_golden_spans_and_batches():
    for pages, pb, field, exp in GOLDEN["spans"]:
        got = _or_none(lambda: [list(s) for s in page_spans(pages, pb, field)])
        assert got == exp
    for seqs, cap, budget, context, exp in GOLDEN["batches"]:
        got = _or_none(lambda: SequenceBatch.make(seqs, cap, budget, context))
        if exp is None:
            assert got is None
        else:
            assert got is not None
            for k, v in exp.items():
                assert getattr(got, k) == v, k
