"""GPU parity of packed-MLA attention over query rows (BF16 windows over ring
page tables, C8 sparse index lists, learned sinks) against the CPU oracle,
bf16 outputs within 1e-2 abs + 1e-2 rel. Fixtures follow the reference probes
(native/probes/sliding_window_probe.cpp:85-163, packed_cache_probe.cpp:18-66)
plus random multi-sequence batches that cross partitions."""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_close, bf16_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu
f32 = np.float32
SCALE = 1.0 / math.sqrt(192.0)


def bf(x):
    return W.bf16_bits(np.asarray(x, np.float32))


def run(q, cache, table, kv, max_context, cu=None, idx=None, window=0, sk=None, sv=None):
    import torch
    from ironpangu_amd import ops
    c8 = cache.dtype == np.uint8
    bs = cache.shape[1]
    out = ops.mla_attention(to_dev(q), to_dev(cache), to_dev(np.asarray(table, np.int32)),
                            to_dev(np.asarray(kv, np.int32)), max_context,
                            cu_seqlens=None if cu is None else to_dev(np.asarray(cu, np.int32)),
                            indices=None if idx is None else to_dev(np.asarray(idx, np.int32)),
                            window=window, sink_keys=None if sk is None else to_dev(sk),
                            sink_values=None if sv is None else to_dev(sv))
    torch.cuda.synchronize()
    flat = cache.reshape(-1, 656 if c8 else 576)
    exp = oracle.mla_attention(q, flat, table, kv, q.shape[1], bs, SCALE, c8=c8, cu_seqlens=cu,
                               indices=idx, window=window, sink_k=sk, sink_v=sv)
    return bf16_host(out), exp


def sinks(n, seed):
    rng = np.random.default_rng(seed)
    sk = bf(rng.standard_normal((n, 576)).astype(f32) * f32(0.5))
    sv = bf(rng.standard_normal((n, 512)).astype(f32) * f32(0.5))
    return sk, sv


@pytest.mark.parametrize("rows", [1, 4, 16])
def test_window_ring_probe(rows):
    from ironpangu_amd.host import WindowLayout
    window, page = 512, 16
    chunk = max(rows, 4)
    lay = WindowLayout(65536, window, chunk, page)  # sliding_window_probe.cpp:85
    pages = lay.physical_pages
    table = lay.table()[None, :]
    hq = bf(((np.arange(rows * 6 * 512) * 7) % 97 - 48).astype(f32) / f32(128)).reshape(rows, 6, 512)
    hqr = bf(((np.arange(rows * 6 * 64) * 11) % 89 - 44).astype(f32) / f32(128)).reshape(rows, 6, 64)
    hs = bf(((np.arange(128 * 512) * 19) % 103 - 51).astype(f32) / f32(128)).reshape(128, 512)
    hsr = bf(((np.arange(128 * 64) * 23) % 107 - 53).astype(f32) / f32(128)).reshape(128, 64)
    q = np.ascontiguousarray(np.concatenate([hq, hqr], axis=2))
    sk = np.ascontiguousarray(np.concatenate([hs, hsr], axis=1))
    for start in (0, 15, 509, 525, 4095, 65536 - chunk):
        cache = np.full((pages * page, 576), bf([4.0])[0], np.uint16)  # poison outside the window
        pos = np.arange(max(0, start - window + 1), start + chunk)
        d = np.arange(576)
        cache[lay.slots(pos)] = bf(
            ((pos[:, None] * 17 + d[None, :] * 13) % 101 - 50).astype(f32) / f32(128))
        got, exp = run(q, cache.reshape(pages, page, 576), table, [start + rows], 65536,
                       cu=[0, rows], window=window, sk=sk, sv=hs)
        assert_close(got, exp, what=f"start {start}")


@pytest.mark.parametrize("rows", [1, 4, 16])
def test_sparse_c8_probe(rows):
    r = np.arange(512)[:, None]
    d = np.arange(576)[None, :]
    x = bf(np.where(r == 0, 0, ((r * 7 + d * 11) % 97 - 48).astype(f32) * (1 + d // 128) / f32(128)))
    cache = np.zeros((512, 656), np.uint8)
    oracle.mla_norm_rope_write(x, bf(np.ones(512, f32)), bf(np.full((512, 64), 0.8, f32)),
                               bf(np.full((512, 64), 0.6, f32)), np.arange(512), cache, True)
    q = bf(((np.arange(rows * 6 * 576) * 13) % 101 - 50).astype(f32) / f32(128)).reshape(rows, 6, 576)
    hs = bf(((np.arange(128 * 576) * 19) % 103 - 51).astype(f32) / f32(128)).reshape(128, 576)
    hv = np.ascontiguousarray(hs[:, :512])
    table = np.arange(16, dtype=np.int32)[None, :]
    for end in (rows - 1, 31, 32, 511):
        idx = np.array([[i if i <= end - rows + 1 + t else -1 for i in range(512)]
                        for t in range(rows)], np.int32)
        got, exp = run(q, cache.reshape(16, 32, 656), table, [end + 1], 512, cu=[0, rows], idx=idx,
                       sk=hs, sv=hv)
        assert_close(got, exp, what=f"end {end}")


def batch(seed, counts, kv, bs, heads, c8):
    """Packed batch: sequence s has counts[s] query rows and kv[s] cached keys."""
    rng = np.random.default_rng(seed)
    kv = np.asarray(kv, np.int32)
    need = (kv.astype(np.int64) + bs - 1) // bs
    pool = int(need.sum()) + 8
    stride = int(need.max()) + 2
    table = W.block_tables_for(rng, kv, bs, pool, stride)
    rows = int(sum(counts))
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    q = bf(rng.standard_normal((rows, heads, 576)).astype(f32) * f32(0.5))
    lat = bf(rng.standard_normal((pool * bs, 576)).astype(f32) * f32(0.5))
    cache = oracle.mla_pack_c8(lat).reshape(pool, bs, 656) if c8 else lat.reshape(pool, bs, 576)
    return q, cache, table, kv, cu, stride * bs


@pytest.mark.parametrize("window,bs,with_sinks", [(0, 64, False), (0, 32, True), (37, 64, True),
                                                  (600, 32, False), (2500, 128, True)])
def test_window_batches(window, bs, with_sinks):
    counts = [1, 7, 1, 33, 2]
    kv = [5000, 300, 1, 2100, 40]
    q, cache, table, kv, cu, maxc = batch(5, counts, kv, bs, 12, False)
    sk, sv = sinks(128, 6) if with_sinks else (None, None)
    got, exp = run(q, cache, table, kv, maxc, cu=cu, window=window, sk=sk, sv=sv)
    assert_close(got, exp)


@pytest.mark.parametrize("topk,bs,n_sinks", [(2048, 32, 128), (512, 64, 0), (3000, 64, 17)])
def test_sparse_batches(topk, bs, n_sinks):
    counts = [3, 1, 6]
    kv = [4000, 900, 2200]
    q, cache, table, kv, cu, maxc = batch(7, counts, kv, bs, 16, True)
    rng = np.random.default_rng(8)
    rows = int(sum(counts))
    idx = np.full((rows, topk), -1, np.int32)
    for s in range(len(counts)):
        for t in range(cu[s], cu[s + 1]):
            causal = kv[s] - counts[s] + (t - cu[s]) + 1
            n = min(causal, topk)
            idx[t, :n] = rng.choice(causal, size=n, replace=False)  # distinct, any order
    sk, sv = sinks(n_sinks, 9) if n_sinks else (None, None)
    got, exp = run(q, cache, table, kv, maxc, cu=cu, idx=idx, sk=sk, sv=sv)
    assert_close(got, exp)


@pytest.mark.parametrize("with_sinks", [False, True])
def test_rows_without_keys(with_sinks):
    # sequence 1 has no cached key (kv 0): zeros, or sink-only attention
    q, cache, table, kv, cu, maxc = batch(11, [1, 1, 2], [70, 1, 90], 32, 8, False)
    kv = np.array([70, 0, 90], np.int32)
    sk, sv = sinks(5, 12) if with_sinks else (None, None)
    got, exp = run(q, cache, table, kv, maxc, cu=cu, sk=sk, sv=sv)
    assert_close(got, exp)
    if not with_sinks:
        assert not got[1].any()


def test_decode_entry_matches_general():
    import torch
    from ironpangu_amd import ops
    q, cache, table, kv, cu, maxc = batch(13, [1] * 6, [3000, 1, 64, 2049, 700, 4096], 64, 16, False)
    a = ops.mla_decode(to_dev(q), to_dev(cache), to_dev(table), to_dev(kv), maxc)
    b = ops.mla_attention(to_dev(q), to_dev(cache), to_dev(table), to_dev(kv), maxc)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("c8,with_sinks,window", [(False, False, 0), (True, True, 0), (False, True, 300)])
def test_many_rows(c8, with_sinks, window):
    """More than 1024 query rows: the plan walks the rows in chunks of 1024
    (partition slots and full-partition positions carried between chunks).
    C8 rows take index lists (top-300 of their causal keys)."""
    rng = np.random.default_rng(21)
    counts = [1] * 1290 + [3, 1, 5]
    kv = np.concatenate([rng.integers(0, 160, 1290), [2900, 3100, 1700]]).astype(np.int32)
    kv[:1290:97] = rng.integers(1000, 2600, len(kv[:1290:97]))  # some rows span several partitions
    q, cache, table, kv, cu, maxc = batch(23, counts, kv, 32, 4, c8)
    sk, sv = sinks(9, 24) if with_sinks else (None, None)
    idx = None
    if c8:
        topk = 300
        idx = np.full((int(sum(counts)), topk), -1, np.int32)
        for s in range(len(counts)):
            for t in range(cu[s], cu[s + 1]):
                causal = int(kv[s]) - counts[s] + (t - cu[s]) + 1
                n = min(max(causal, 0), topk)
                idx[t, :n] = rng.choice(max(causal, 1), size=n, replace=False)
    got, exp = run(q, cache, table, kv, maxc, cu=cu, idx=idx, window=window, sk=sk, sv=sv)
    assert_close(got, exp)


@pytest.mark.parametrize("rows,c8", [(256, False), (257, False), (256, True), (257, True)])
def test_self_plan_row_limit(rows, c8):
    """Calls of at most 256 rows plan inside the attention workgroups, larger
    ones through the plan launch: both sides of the limit, with sinks, rows
    without keys and rows spread over several shares (C8 rows take top-200
    index lists)."""
    rng = np.random.default_rng(31 + rows)
    counts = [1] * (rows - 4) + [2, 2]
    kv = rng.integers(0, 900, len(counts)).astype(np.int32)
    kv[::41] = 0                                                   # rows without keys
    # rows over several shares; bf16 calls stay below the 2^18 possible keys
    # (rows x max_context) of the two-workgroup layout, which plans through
    # the plan launch whatever the row count
    kv[5::37] = rng.integers(2500, 4000, len(kv[5::37])) if c8 else rng.integers(600, 900, len(kv[5::37]))
    q, cache, table, kv, cu, maxc = batch(29, counts, kv, 32, 16, c8)
    assert c8 or rows * maxc < 1 << 18
    sk, sv = sinks(40, 12)
    idx = None
    if c8:
        topk = 200
        idx = np.full((int(sum(counts)), topk), -1, np.int32)
        for s in range(len(counts)):
            for t in range(cu[s], cu[s + 1]):
                causal = int(kv[s]) - counts[s] + (t - cu[s]) + 1
                n = min(max(causal, 0), topk)
                idx[t, :n] = rng.choice(max(causal, 1), size=n, replace=False)
    got, exp = run(q, cache, table, kv, maxc, cu=cu, idx=idx, sk=sk, sv=sv)
    assert_close(got, exp)


@pytest.mark.parametrize("c8,with_sinks", [(False, False), (False, True), (True, False)])
def test_merge_partial_counts(c8, with_sinks):
    """One row split over 6 to 11 shares (at least 512 units per share): the
    merge's one-round-trip path (at most 8 partials, counting the sink
    partial) and its general path on both sides of the limit. C8 rows go
    through the dense decode entry (the general entry takes index lists)."""
    import torch
    from ironpangu_amd import ops
    sk, sv = sinks(128, 31) if with_sinks else (None, None)
    for kv in (2900, 3300, 3552, 3800, 4064, 4400, 4700, 5400):
        q, cache, table, kvs, cu, maxc = batch(kv, [1], [kv], 64, 16, c8)
        if c8:
            out = ops.mla_decode(to_dev(q), to_dev(cache), to_dev(table), to_dev(kvs), maxc)
            torch.cuda.synchronize()
            got = bf16_host(out)
            exp = oracle.mla_decode(q, cache.reshape(-1, 656), table, kvs, 16, 64, SCALE, c8=True)
        else:
            got, exp = run(q, cache, table, kvs, maxc, cu=cu, sk=sk, sv=sv)
        assert_close(got, exp, what=f"kv {kv}")


@pytest.mark.parametrize("rows", [300, 130])
def test_dense_c8_weighted_shares(rows):
    """Dense C8 decode calls large enough for the full persistent grid, where
    each CU's three workgroups take shares weighted by dispatch order: 300 rows
    plan through the plan launch, 130 inside the workgroups. The rows' tables
    reuse a small pool of physical blocks (reads only), so the call is large
    while the cache stays small; lengths straddle share boundaries at random."""
    import torch
    from ironpangu_amd import ops
    print(f"dense c8 weighted shares rows={rows}", flush=True)
    rng = np.random.default_rng(41 + rows)
    bs, pool, heads = 64, 192, 16
    kv = rng.integers(2000, 8000 if rows < 256 else 4000, rows).astype(np.int32)
    kv[::17] = rng.integers(1, 300, len(kv[::17]))  # short rows inside one share
    stride = int((kv.max() + bs - 1) // bs) + 1
    table = rng.integers(0, pool, (rows, stride)).astype(np.int32)
    lat = bf(rng.standard_normal((pool * bs, 576)).astype(f32) * f32(0.5))
    cache = oracle.mla_pack_c8(lat).reshape(pool, bs, 656)
    q = bf(rng.standard_normal((rows, heads, 576)).astype(f32) * f32(0.5))
    out = ops.mla_decode(to_dev(q), to_dev(cache), to_dev(table), to_dev(kv), stride * bs)
    torch.cuda.synchronize()
    exp = oracle.mla_decode(q, cache.reshape(-1, 656), table, kv, heads, bs, SCALE, c8=True)
    assert_close(bf16_host(out), exp)


@pytest.mark.parametrize("with_sinks", [False, True])
def test_wide_layout_in_kernel_plan(with_sinks):
    """Dense bf16 calls of at most 256 rows in the two-workgroup layout (rows x
    max_context >= 2^18) plan inside the attention workgroups, into the plan
    arrays: packed multi-row sequences, rows without keys, rows over several
    shares, with and without sinks, against the oracle."""
    print(f"wide in-kernel plan sinks={with_sinks}", flush=True)
    rng = np.random.default_rng(53 + with_sinks)
    counts = [1] * 30 + [3, 2, 4]
    kv = rng.integers(0, 700, len(counts)).astype(np.int32)
    kv[::7] = 0                                                   # rows without keys
    kv[3::9] = rng.integers(4000, 7000, len(kv[3::9]))           # rows over several shares
    kv[-3:] = [5000, 900, 6100]
    q, cache, table, kv, cu, maxc = batch(61, counts, kv, 64, 16, False)
    assert int(sum(counts)) * maxc >= 1 << 18 and int(sum(counts)) <= 256
    sk, sv = sinks(128, 62) if with_sinks else (None, None)
    got, exp = run(q, cache, table, kv, maxc, cu=cu, sk=sk, sv=sv)
    assert_close(got, exp)
