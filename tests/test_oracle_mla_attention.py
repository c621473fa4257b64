"""Pins for the general packed-MLA attention of the CPU oracle
(oracle_mla_attention): the fixtures and acceptance rules of the reference's
two probes restated in float64 here —
native/probes/packed_cache_probe.cpp:18-66 (C8 rows from the fused writer,
causal index lists with -1 padding, 128 learned sinks, tolerance .003 + .02|e|)
and native/probes/sliding_window_probe.cpp:85-163 (BF16 rows in a ring of
physical pages, window 512, 128 sinks, tolerance .001 + .02|e|) — plus
agreement with oracle_mla_decode and invariances of the sparse lists."""
import math

import numpy as np
import pytest

import oracle
from ironpangu_amd import workloads as W

f32 = np.float32
SCALE = 1.0 / math.sqrt(192.0)


def bf(x):
    return W.bf16_bits(np.asarray(x, np.float32))


def fp(b):
    return W.bf16_to_f32(b).astype(np.float64)


def softmax_ref(qh, keys, vals):
    s = keys @ qh * SCALE
    e = np.exp(s - s.max())
    return (e / e.sum()) @ vals


# ---------------------------------------------------------------- packed C8 probe

def packed_probe_case(rows):
    """packed_cache_probe.cpp:18-23,49-53: 512 cache rows (row 0 zero), C8 writer with
    gamma 1, cos .8, sin .6; q[i] = bf16((i*13 % 101 - 50)/128) [rows,6,576]; sinks
    bf16((i*19 % 103 - 51)/128) [128,576], values = their first 512; table 0..15, page 32."""
    r = np.arange(512)[:, None]
    d = np.arange(576)[None, :]
    x = bf(np.where(r == 0, 0, ((r * 7 + d * 11) % 97 - 48).astype(f32) * (1 + d // 128) / f32(128)))
    cache = np.zeros((512, 656), np.uint8)
    oracle.mla_norm_rope_write(x, bf(np.ones(512, f32)), bf(np.full((512, 64), 0.8, f32)),
                               bf(np.full((512, 64), 0.6, f32)), np.arange(512), cache, True)
    q = bf(((np.arange(rows * 6 * 576) * 13) % 101 - 50).astype(f32) / f32(128)).reshape(rows, 6, 576)
    hs = bf(((np.arange(128 * 576) * 19) % 103 - 51).astype(f32) / f32(128)).reshape(128, 576)
    return cache, q, hs, np.ascontiguousarray(hs[:, :512])


def unpack(cache):
    lat = cache[:, :512].view(np.int8).astype(np.float64)
    sc = cache[:, 640:656].copy().view(np.float32).astype(np.float64)
    lat = lat * np.repeat(sc, 128, axis=1)
    rope = fp(cache[:, 512:640].copy().view(np.uint16))
    return np.concatenate([lat, rope], axis=1)


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_packed_probe(rows):
    cache, q, hs, hv = packed_probe_case(rows)
    full = unpack(cache)
    table = np.arange(16, dtype=np.int32)[None, :]
    for end in (rows - 1, 31, 32, 511):
        idx = np.array([[i if i <= end - rows + 1 + t else -1 for i in range(512)]
                        for t in range(rows)], np.int32)
        got = oracle.mla_attention(q, cache, table, [end + 1], 6, 32, SCALE, c8=True,
                                   cu_seqlens=[0, rows], indices=idx, sink_k=hs, sink_v=hv)
        for t in range(rows):
            pos = end - rows + 1 + t
            keys = np.concatenate([full[:pos + 1], fp(hs)])
            vals = np.concatenate([full[:pos + 1, :512], fp(hv)])
            for h in range(6):
                exp = softmax_ref(fp(q[t, h]), keys, vals)
                assert (np.abs(got[t, h] - exp) <= 0.003 + 0.02 * np.abs(exp)).all(), (end, t, h)


# ---------------------------------------------------------------- BF16 window probe

def window_layout(window, chunk, page=16, context=65536):
    """SlidingWindowLayout (sliding_window_layout.h:9-33): physical pages retained
    and the table of absolute logical pages -> physical page (logical % pages)."""
    retained = window + chunk - 1
    pages = min((retained + page - 2) // page + 1, (context + page - 1) // page)
    entries = (context + page - 1) // page
    return pages, (np.arange(entries) % pages).astype(np.int32)


def key(pos, d):
    return bf(((np.asarray(pos)[:, None].astype(np.int64) * 17 + np.asarray(d)[None, :] * 13) % 101
               - 50).astype(f32) / f32(128))


@pytest.mark.parametrize("rows", [1, 4])
def test_window_probe(rows):
    window, page = 512, 16
    chunk = max(rows, 4)
    pages, table = window_layout(window, chunk)
    hq = bf(((np.arange(rows * 6 * 512) * 7) % 97 - 48).astype(f32) / f32(128)).reshape(rows, 6, 512)
    hqr = bf(((np.arange(rows * 6 * 64) * 11) % 89 - 44).astype(f32) / f32(128)).reshape(rows, 6, 64)
    hs = bf(((np.arange(128 * 512) * 19) % 103 - 51).astype(f32) / f32(128)).reshape(128, 512)
    hsr = bf(((np.arange(128 * 64) * 23) % 107 - 53).astype(f32) / f32(128)).reshape(128, 64)
    q = np.concatenate([hq, hqr], axis=2)
    sk = np.concatenate([hs, hsr], axis=1)
    for start in (0, 15, 509, 525, 4095):
        last = rows - 1
        # Only the retained union is materialised; other storage is poison (bf16 4.0).
        cache = np.full((pages * page, 576), bf([4.0])[0], np.uint16)
        lo = max(0, start - window + 1)
        pos = np.arange(lo, start + chunk)
        slots = table[pos // page] * page + pos % page
        assert len(np.unique(slots)) == len(slots), "window overwrote a live row"
        cache[slots] = key(pos, np.arange(576))
        got = oracle.mla_attention(q, cache, table[None, :], [start + last + 1], 6, page, SCALE,
                                   cu_seqlens=[0, rows], window=window, sink_k=sk, sink_v=hs)
        for t in range(rows):
            p = start + last - rows + 1 + t
            first = max(0, p - window + 1)
            kp = np.arange(first, p + 1)
            keys = np.concatenate([fp(key(kp, np.arange(576))), fp(sk)])
            vals = np.concatenate([fp(key(kp, np.arange(512))), fp(hs)])
            for h in range(6):
                exp = softmax_ref(fp(q[t, h]), keys, vals)
                assert (np.abs(got[t, h] - exp) <= 0.001 + 0.02 * np.abs(exp)).all(), (start, t, h)


# ---------------------------------------------------------------- consistency

def small_case(seed=0, c8=False):
    case = W.mla_host_case(seed, num_seqs=4, lo=1, hi=300, dist="uniform", heads=6, block_size=32)
    cache = case.host["pool"]
    if c8:
        cache = oracle.mla_pack_c8(cache)
    return case, cache


@pytest.mark.parametrize("c8", [False, True])
def test_dense_rows_match_decode(c8):
    case, cache = small_case(1, c8)
    h = case.host
    a = oracle.mla_decode(h["q"], cache, case.block_tables, case.seq_lens, 6, 32, case.scale, c8=c8)
    b = oracle.mla_attention(h["q"], cache, case.block_tables, case.seq_lens, 6, 32, case.scale, c8=c8)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("c8", [False, True])
def test_sparse_list_equals_dense_and_order_free(c8):
    case, cache = small_case(2, c8)
    h = case.host
    topk = int(case.seq_lens.max()) + 5
    rng = np.random.default_rng(3)
    idx = np.full((4, topk), -1, np.int32)
    perm = np.full((4, topk), -1, np.int32)
    for s, L in enumerate(case.seq_lens):
        idx[s, :L] = np.arange(L)
        perm[s, :L] = rng.permutation(L)
    dense = oracle.mla_attention(h["q"], cache, case.block_tables, case.seq_lens, 6, 32, case.scale, c8=c8)
    sp = oracle.mla_attention(h["q"], cache, case.block_tables, case.seq_lens, 6, 32, case.scale,
                              c8=c8, indices=idx)
    sq = oracle.mla_attention(h["q"], cache, case.block_tables, case.seq_lens, 6, 32, case.scale,
                              c8=c8, indices=perm)
    assert np.allclose(dense, sp, atol=1e-6, rtol=1e-5)
    assert np.allclose(dense, sq, atol=1e-5, rtol=1e-4)


def test_window_is_a_suffix_and_rows_follow_causal_rule():
    case, cache = small_case(4)
    h = case.host
    lens = case.seq_lens.copy()
    win = 17
    a = oracle.mla_attention(h["q"], cache, case.block_tables, lens, 6, 32, case.scale, window=win)
    # same result from an explicit index list of the last `win` positions
    idx = np.full((4, win), -1, np.int32)
    for s, L in enumerate(lens):
        k = min(L, win)
        idx[s, :k] = np.arange(L - k, L)
    b = oracle.mla_attention(h["q"], cache, case.block_tables, lens, 6, 32, case.scale, indices=idx)
    assert np.allclose(a, b, atol=1e-6, rtol=1e-5)
    # packed rows: row t of a 3-row chunk equals a decode row with kv_len - 2 + t keys
    q3 = np.repeat(h["q"][:1], 3, axis=0)
    c = oracle.mla_attention(q3, cache, case.block_tables[:1], lens[:1], 6, 32, case.scale,
                             cu_seqlens=[0, 3])
    for t in range(3):
        d = oracle.mla_attention(h["q"][:1], cache, case.block_tables[:1], lens[:1] - 2 + t, 6, 32,
                                 case.scale)
        assert np.array_equal(c[t], d[0])
