"""The compact-pool remapping that the full-size GPU tests use for their host
check: attention over the compact copy equals attention over the whole pool."""
import numpy as np

import oracle
from helpers import compact_blocks, remap_slots
from ironpangu_amd import workloads as W


def test_compact_pool_preserves_decode():
    case = W.decode_host_case(21, num_seqs=7, lo=1, hi=700, dist="uniform", q_heads=8,
                              kv_heads=2, head_dim=64, block_size=32, pool_blocks=200)
    h = case.host
    used, ctab = compact_blocks(case.block_tables, case.seq_lens, 32)
    kp = h["k_pool"].reshape(200, 32, 2, 64)
    vp = h["v_pool"].reshape(200, 32, 2, 64)
    full = oracle.paged_decode(h["q"], kp, vp, case.block_tables, case.seq_lens, 8, 2, 64, 32,
                               case.scale)
    comp = oracle.paged_decode(h["q"], kp[used], vp[used], ctab, case.seq_lens, 8, 2, 64, 32,
                               case.scale)
    assert np.array_equal(full, comp)
    assert used.size == int(((case.seq_lens + 31) // 32).sum())
    cs = remap_slots(case.slot_mapping, used, 32)
    assert np.array_equal(kp.reshape(-1, 128)[case.slot_mapping], kp[used].reshape(-1, 128)[cs])
