"""Sliding-window page ring (host.WindowLayout, include/ifattn_host.h) against
the reference's own acceptance test restated
(native/probes/sliding_window_layout_test.cpp:10-38) and, where the reference
tree was present at build time, against SlidingWindowLayout compiled in place
(oracle/_ref)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from ironpangu_amd.host import MetadataError, WindowLayout


@pytest.mark.parametrize("width", [1, 4, 16, 32])
def test_no_live_row_overwritten(width):
    """Every chunk start of a 65536-token context: the window (511 earlier rows)
    plus the chunk never share a physical row, and the table agrees with the
    write (sliding_window_layout_test.cpp:12-27), checked for all starts at once."""
    lay = WindowLayout(65536, 512, width, 16)
    pos = np.arange(65536)
    slots = lay.slots(pos)
    table = lay.table()
    assert np.array_equal(slots // 16, table[pos // 16]), "table and write disagree"
    assert slots.max() < lay.physical_pages * 16
    # live set at chunk start s is the interval [max(0, s-511), s+width): it is
    # collision-free iff equal rows recur no closer than 511 + width positions.
    order = np.lexsort((pos, slots))
    same = slots[order][1:] == slots[order][:-1]
    gaps = np.diff(pos[order])[same]
    assert gaps.min() >= 511 + width
    with pytest.raises(MetadataError):
        lay.append(65536)
    with pytest.raises(MetadataError):
        lay.physical_page(lay.table_entries)


@pytest.mark.parametrize("context", [1, 15, 16, 17, 129, 512])
def test_short_context_not_overallocated(context):
    assert WindowLayout(context, 512, 1, 16).physical_pages == (context + 15) // 16


@pytest.mark.parametrize("args", [(0, 512, 4, 16), (65536, 0, 4, 16), (65536, 512, 0, 16),
                                  (65536, 512, 4, 0), (1, 512, 4, 16),
                                  (2**32 - 1, 2**32 - 1, 1, 16)])
def test_invalid_layouts_rejected(args):
    with pytest.raises(MetadataError):
        WindowLayout(*args)


def test_owned_pages_follow_the_ring():
    lay = WindowLayout(4096, 512, 16, 16)
    owned = np.arange(lay.physical_pages)[::-1] * 3 + 100
    t = lay.table(owned)
    assert np.array_equal(t, owned[np.arange(lay.table_entries) % lay.physical_pages])
    s = lay.slots([0, 17, 4095], owned)
    assert s.tolist() == [owned[0] * 16, owned[1] * 16 + 1, owned[255 % lay.physical_pages] * 16 + 15]
    with pytest.raises(MetadataError):
        lay.table(owned[:-1])
    with pytest.raises(MetadataError):
        lay.table(np.r_[owned[:-1], owned[0]])


def test_matches_reference_build():
    ref = oracle.ref()
    if ref is None:
        pytest.skip("reference tree absent at build time: oracle/_ref not built")
    rng = np.random.default_rng(5)
    for context, window, chunk, page in [(65536, 512, 4, 16), (65536, 2048, 32, 16), (1000, 512, 7, 32),
                                         (129, 512, 1, 16), (300000, 4096, 2048, 64)]:
        lay = WindowLayout(context, window, chunk, page)
        pages, entries = C.c_uint32(), C.c_uint32()
        assert ref.ref_window_layout(context, window, chunk, page, C.byref(pages), C.byref(entries)) == 0
        assert (lay.physical_pages, lay.table_entries) == (pages.value, entries.value)
        pos = rng.integers(0, context, 200)
        mine = lay.slots(pos)
        for p, m in zip(pos, mine):
            s = C.c_uint32()
            assert ref.ref_window_append(context, window, chunk, page, int(p), C.byref(s)) == 0
            assert s.value == m
