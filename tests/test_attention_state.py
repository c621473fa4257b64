"""The attention-state object (include/ifattn_state.h), the counterpart of the
reference's AttentionState (native/src/openpangu_decoder_state.h:16-48):
geometry of each cache format, and append / blocks against the reference's own
page binding (native/src/page_binding.h, compiled in place under oracle/_ref)
driven through the same operations. Host-only: no device buffer is touched."""
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from ironpangu_amd.host import AttentionState, MetadataError

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))


def test_geometry_of_each_format():
    # openpangu_decoder_state.h:24-29: packed C8 [res*cap/32, 32, 1, 656] int8,
    # bf16 [res*cap/16, 16, 1, 576], row-quantized [cap*576*bits/8] bytes;
    # table [1, packed ? cap/32 : (context ? ceil(context/16) : cap/16)].
    s = AttentionState(16, 512, False, 2, True, 0, 6)
    assert s.format == "bf16" and s.geometry["num_blocks"] == 64 and s.geometry["table_entries"] == 32
    assert s.geometry["cache_bytes"] == 64 * 16 * 1152
    s = AttentionState(16, 4096, True, 3, False, 0, 6)
    assert s.format == "packed_c8" and s.geometry["num_blocks"] == 384
    assert s.geometry["table_entries"] == 128 and s.geometry["cache_bytes"] == 384 * 32 * 656
    s = AttentionState(16, 8192, False, 1, False, 65536, 6)
    assert s.geometry["table_entries"] == 4096 and s.geometry["num_blocks"] == 512
    s = AttentionState(8, 512, False, 1, False, 0, 6)
    assert s.format == "row_quant" and s.geometry["cache_bytes"] == 512 * 576
    s = AttentionState(4, 512, False, 1, False, 0, 6)
    assert s.geometry["cache_bytes"] == 512 * 288


def test_rejections():
    with pytest.raises(MetadataError):
        AttentionState(8, 512, False, 2, False, 0, 6)    # resident row-quantized cache
    with pytest.raises(MetadataError):
        AttentionState(12, 512, False, 1, False, 0, 6)   # bits
    with pytest.raises(MetadataError):
        AttentionState(16, 500, False, 1, False, 0, 6)   # capacity not whole pages
    with pytest.raises(MetadataError):
        AttentionState(16, 512, False, 1, False, 0, 17)  # heads
    s = AttentionState(16, 512, False, 1, False, 4096, 6)
    with pytest.raises(MetadataError):
        s.append(4096)                                   # absolute position past the context


@pytest.mark.parametrize("packed,context,shared", [(False, 0, False), (False, 4096, True),
                                                   (True, 0, True), (True, 2048, False)])
def test_append_and_blocks_match_reference_page_binding(packed, context, shared):
    from make_golden import RefPages
    if oracle.ref() is None:
        pytest.skip("reference host metadata not built (reference tree absent at build time)")
    cap, residents, page = 1024, 3, 32 if packed else 16
    s = AttentionState(16, cap, packed, residents, shared, context, 6)
    ref = RefPages(page, cap, residents, shared)
    entries = s.geometry["table_entries"]
    rng = np.random.default_rng(7 + int(packed) + context)
    per = cap // page
    for step in range(6):
        slot = int(rng.integers(0, residents))
        s.page_binding.select(slot)
        ref.select(slot)
        if shared and step % 2:
            s.page_binding.release(slot)
            ref.release(slot)
            free = [p for p in range(per * residents)
                    if all(p not in s.page_binding.pages(r) for r in range(residents))]
            ids = list(rng.permutation(free)[: int(rng.integers(1, per + 1))].astype(int))
        else:
            ids = list(rng.permutation(per).astype(int) + slot * per) if not shared else \
                list(s.page_binding.pages(slot)[::-1]) or [int(slot * per)]
        if not shared or ids:
            s.page_binding.bind(ids)
            assert ref.bind(np.array(ids, np.int32)) == 0
        for pos in rng.integers(0, context or cap, 20):
            pos = int(pos)
            p = pos % cap if context else pos
            exp = ref.append(slot, p)
            if exp is None:
                with pytest.raises(MetadataError):
                    s.append(pos)
            else:
                assert s.append(pos) == exp
        exp_t = ref.batch_table([slot], entries, context != 0)
        assert exp_t is not None and s.blocks().tolist() == exp_t
