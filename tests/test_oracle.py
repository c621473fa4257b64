"""Pins for the CPU oracle (oracle/oracle.cpp): each function is checked
against closed forms, the reference's own probe vectors, or invariants chosen
so that a plausible mistake (wrong GQA grouping, wrong causal offset, wrong
scale, transposed operands, dropped rope term, wrong rounding) fails."""
import math

import numpy as np
import pytest

import oracle
from ironpangu_amd import workloads as W

f32 = np.float32


def bf(x):
    return W.bf16_bits(np.asarray(x, np.float32))


def test_kv_write_touches_only_mapped_rows():
    rng = np.random.default_rng(0)
    cache = rng.integers(0, 65535, size=(64, 4, 8), dtype=np.uint16)
    before = cache.copy()
    rows = rng.integers(0, 65535, size=(5, 4, 8), dtype=np.uint16)
    slots = np.array([3, 60, -1, 17, 64], np.int64)  # -1 and 64 are skipped
    oracle.kv_write(rows, cache, slots)
    for r, s in enumerate(slots):
        if 0 <= s < 64:
            assert np.array_equal(cache[s], rows[r])
    untouched = np.setdiff1d(np.arange(64), slots[(slots >= 0) & (slots < 64)])
    assert np.array_equal(cache[untouched], before[untouched])


def test_quant_rows_probe_vector_and_ties():
    # native/probes/cache_quantization_probe.cpp:17: x[j] = bf16((j % 61 - 30) / 13)
    x = bf(((np.arange(576) % 61) - 30).astype(f32) / f32(13))
    codes, scales = oracle.quant_rows(x, 576)
    xf = W.bf16_to_f32(x)
    assert abs(scales[0] - np.abs(xf).max() / 127) <= 1e-6
    assert np.array_equal(codes[0], np.rint(xf / scales[0]).astype(np.int8))  # rint = half even
    row = bf([127, 0.5, 1.5, 2.5, -0.5, -2.5, 3.5, -127])
    c, s = oracle.quant_rows(row, 8)
    assert s[0] == 1.0 and c[0].tolist() == [127, 0, 2, 2, 0, -2, 4, -127]
    z, zs = oracle.quant_rows(np.zeros(16, np.uint16), 16, zero_scale=1.0)
    assert zs[0] == 1.0 and not z.any()


def test_quant_legacy_ties_away_and_int4_nibbles():
    row = bf([127, 0.5, 1.5, 2.5, -0.5, -2.5, 3.5, -127])
    packed, scale = oracle.quant_legacy(row, 8)
    assert scale == 1.0 and packed.view(np.int8).tolist() == [127, 1, 2, 3, -1, -3, 4, -127]
    p4, s4 = oracle.quant_legacy(bf([7, -7, 1, -1, 0, 3.5, -3.5, 2]), 4)
    assert s4 == 1.0
    # low nibble first, two's complement: (7,-7)->0x97, (1,-1)->0xF1, (0,3.5->4)->0x40, (-4,2)->0x2C
    assert p4.tolist() == [0x97, 0xF1, 0x40, 0x2C]
    zero, zs = oracle.quant_legacy(np.zeros(8, np.uint16), 8)
    assert zs == 1.0 and not zero.any()


def test_dequant_legacy_rows_after_position_are_zero():
    packed = np.arange(4 * 8, dtype=np.uint8)
    scales = np.array([0.5, 2.0, 4.0, 8.0], np.float32)
    out = oracle.dequant_legacy(packed, scales, 1, 8, 8).reshape(4, 8)
    assert not out[2:].any()
    assert np.array_equal(W.bf16_to_f32(out[1]), (np.arange(8, 16) * 2.0).astype(f32))


def test_mla_pack_c8_probe_checks():
    # packed_cache_probe.cpp:16-45: per-128 tile scale = max/127, codes within
    # one of nearbyint(x/scale) (the oracle is exact), rope copied bit for bit,
    # zero tile -> scale 0 (docs/packed-mla-cache.md:36-37).
    x = np.zeros((3, 576), np.float32)
    r = np.arange(576)
    for row in range(3):
        x[row] = ((row * 7 + r * 11) % 97 - 48) * (1 + r // 128) / 128
    x[1, 256:384] = 0
    bits = bf(x)
    packed = oracle.mla_pack_c8(bits)
    xf = W.bf16_to_f32(bits)
    for row in range(3):
        sc = packed[row, 640:656].view(np.float32)
        for t in range(4):
            tile = xf[row, 128 * t:128 * (t + 1)]
            m = np.abs(tile).max()
            assert sc[t] == np.float32(m / np.float32(127)) if m else sc[t] == 0
            codes = packed[row, 128 * t:128 * (t + 1)].view(np.int8)
            exp = np.rint(tile / sc[t]) if m else np.zeros(128)
            assert np.array_equal(codes, exp.astype(np.int8))
        assert np.array_equal(packed[row, 512:640].view(np.uint16), bits[row, 512:576])


def _decode_case(seed, n=3, hq=8, hkv=2, d=32, bs=32, lo=1, hi=200):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n).astype(np.int32)
    pool = int(((lens + bs - 1) // bs).sum()) + 2
    table = W.block_tables_for(rng, lens, bs, pool, (hi + bs - 1) // bs)
    q = W.bf16_randn(rng, (n, hq, d))
    k = W.bf16_randn(rng, (pool * bs, hkv, d))
    v = W.bf16_randn(rng, (pool * bs, hkv, d))
    return lens, table, q, k, v, pool


def _visible_slots(table, b, length, bs):
    return W.slots_of(table, np.arange(length), np.full(length, b), bs)


def test_decode_q_zero_is_mean_of_values():
    lens, table, q, k, v, _ = _decode_case(1)
    out = oracle.paged_decode(np.zeros_like(q), k, v, table, lens, 8, 2, 32, 32, 0.3)
    vf = W.bf16_to_f32(v)
    for b, L in enumerate(lens):
        mean = vf[_visible_slots(table, b, L, 32)].mean(0)  # [hkv, d]
        for h in range(8):
            np.testing.assert_allclose(out[b, h], mean[h // 4], rtol=1e-5, atol=1e-6)


def test_decode_gqa_grouping_constant_values():
    lens, table, q, k, v, pool = _decode_case(2, hq=12, hkv=3)
    consts = np.array([1.0, -2.0, 4.0], np.float32)
    v = np.broadcast_to(bf(consts)[None, :, None], v.shape).copy()
    out = oracle.paged_decode(q, k, v, table, lens, 12, 3, 32, 32, 0.2)
    for h in range(12):
        np.testing.assert_allclose(out[:, h], consts[h // 4], rtol=1e-6)  # kh = h / group


def test_decode_two_token_softmax_closed_form():
    # tokens 0,1; q = e0, K[0] = a e0, K[1] = b e0, V rows = e0, e1
    d, bs = 32, 32
    q = np.zeros((1, 1, d), np.float32); q[0, 0, 0] = 1
    k = np.zeros((bs, 1, d), np.float32); k[0, 0, 0] = 1.5; k[1, 0, 0] = -0.75
    v = np.zeros((bs, 1, d), np.float32); v[0, 0, 0] = 1; v[1, 0, 1] = 1
    scale = 0.7
    out = oracle.paged_decode(bf(q), bf(k), bf(v), np.array([[0]], np.int32), np.array([2], np.int32),
                              1, 1, d, bs, scale)
    p0 = 1 / (1 + math.exp(scale * (-0.75 - 1.5)))
    assert abs(out[0, 0, 0] - p0) < 1e-6 and abs(out[0, 0, 1] - (1 - p0)) < 1e-6


def test_decode_block_permutation_invariance_and_ref_rounding():
    lens, table, q, k, v, pool = _decode_case(3, lo=40, hi=300)
    out = oracle.paged_decode(q, k, v, table, lens, 8, 2, 32, 32, 0.25)
    perm = np.random.default_rng(9).permutation(pool)
    inv = np.argsort(perm)
    k2 = k.reshape(pool, 32, 2, 32)[inv].reshape(k.shape)  # physical block p moves to perm[p]
    v2 = v.reshape(pool, 32, 2, 32)[inv].reshape(v.shape)
    t2 = perm[table].astype(np.int32)
    out2 = oracle.paged_decode(q, k2, v2, t2, lens, 8, 2, 32, 32, 0.25)
    assert np.array_equal(out, out2)
    # The Rust oracle's bf16 roundings (attention.rs:235,241) stay within its
    # own relative-L2 bound of 0.02 (attention.rs:269) of the fp32 result.
    r = oracle.paged_decode(q, k, v, table, lens, 8, 2, 32, 32, 0.25, ref_rounding=True)
    rel = np.sqrt(((r - out) ** 2).sum() / (out ** 2).sum())
    assert 0 < rel < 0.02


def test_decode_c8_equals_bf16_on_exact_values():
    lens, table, q, k, v, pool = _decode_case(4)
    rng = np.random.default_rng(4)
    kc = rng.integers(-127, 128, size=k.shape).astype(np.int8)
    vc = rng.integers(-127, 128, size=v.shape).astype(np.int8)
    ks = np.full(k.shape[:2], 1 / 64, np.float32)
    vs = np.full(v.shape[:2], 1 / 32, np.float32)
    a = oracle.paged_decode(q, kc, vc, table, lens, 8, 2, 32, 32, 0.3, k_scale=ks, v_scale=vs)
    b = oracle.paged_decode(q, bf(kc.astype(f32) / 64), bf(vc.astype(f32) / 32), table, lens, 8, 2,
                            32, 32, 0.3)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)


def test_prefill_causal_prefix_means_and_decode_row():
    rng = np.random.default_rng(5)
    bs, d = 32, 32
    q_lens = np.array([5, 1, 33], np.int32)
    kv = np.array([70, 40, 33], np.int32)
    pool = int(((kv + bs - 1) // bs).sum()) + 1
    table = W.block_tables_for(rng, kv, bs, pool, 3)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    k = W.bf16_randn(rng, (pool * bs, 2, d))
    v = W.bf16_randn(rng, (pool * bs, 2, d))
    q0 = np.zeros((cu[-1], 8, d), np.uint16)
    out = oracle.varlen_prefill(q0, k, v, table, cu, kv, 8, 2, d, bs, 0.2)
    vf = W.bf16_to_f32(v)
    for s in range(3):
        for t in range(q_lens[s]):
            visible = kv[s] - q_lens[s] + t + 1  # openpangu_attention_metadata.h:22
            mean = vf[_visible_slots(table, s, visible, bs)].mean(0)
            np.testing.assert_allclose(out[cu[s] + t, 5], mean[1], rtol=1e-5, atol=1e-6)
    q = W.bf16_randn(rng, (cu[-1], 8, d))
    out = oracle.varlen_prefill(q, k, v, table, cu, kv, 8, 2, d, bs, 0.2)
    dec = oracle.paged_decode(q[cu[1]:cu[1] + 1], k, v, table[1:2], kv[1:2], 8, 2, d, bs, 0.2)
    np.testing.assert_allclose(out[cu[1]], dec[0], rtol=1e-6)


def test_prefill_nonzero_q_closed_form_per_row():
    """A 3-row chunk after 1 cached token (kv_len 4): row t sees keys
    0 .. t + 1 (kv_len - count + t + 1 of them, openpangu_attention_metadata.h:22).
    q row t and K are multiples of the first unit vector, so score(t, j) =
    scale * c_t * a_j, and V of key j is the constant v_j: every output is a
    small closed-form softmax. A row offset of one either way changes the
    number of visible keys and fails."""
    bs, d, scale = 32, 32, 0.25
    a = np.array([1.0, -2.0, 3.0, 0.5], np.float32)     # K[j] = a_j e0
    vals = np.array([2.0, -1.0, 4.0, 8.0], np.float32)  # V[j] = v_j everywhere
    c = np.array([1.5, -0.75, 2.0], np.float32)         # q row t = c_t e0
    k = np.zeros((bs, 1, d), np.uint16)
    v = np.zeros((bs, 1, d), np.uint16)
    for j in range(4):
        k[j, 0, 0] = bf(a[j])
        v[j, 0, :] = bf(vals[j])
    q = np.zeros((3, 2, d), np.uint16)  # 2 q heads on 1 kv head
    q[:, 0, 0] = bf(c)
    q[:, 1, 0] = bf(-c)
    table = np.zeros((1, 1), np.int32)
    out = oracle.varlen_prefill(q, k, v, table, np.array([0, 3], np.int32),
                                np.array([4], np.int32), 2, 1, d, bs, scale)
    for t in range(3):
        for h, sign in ((0, 1.0), (1, -1.0)):
            n = t + 2
            w = np.exp(scale * sign * c[t] * a[:n].astype(np.float64))
            exp = float((w * vals[:n]).sum() / w.sum())
            np.testing.assert_allclose(out[t, h], exp, rtol=2e-6, atol=1e-6)


def test_mla_q_zero_mean_and_rope_only_scores():
    rng = np.random.default_rng(6)
    bs = 64
    lens = np.array([3, 130], np.int32)
    table = W.block_tables_for(rng, lens, bs, 4, 3)
    rows = W.bf16_randn(rng, (4 * bs, 576), std=0.5)
    out = oracle.mla_decode(np.zeros((2, 4, 576), np.uint16), rows, table, lens, 4, bs, 0.1)
    rf = W.bf16_to_f32(rows)
    for b in range(2):
        mean = rf[_visible_slots(table, b, lens[b], bs), :512].mean(0)
        np.testing.assert_allclose(out[b, 2], mean, rtol=1e-5, atol=1e-6)
    # score from the rope part only: q nonzero only on rope dim 3
    rows2 = np.zeros((4 * bs, 576), np.float32)
    sl = _visible_slots(table, 0, 3, bs)
    rows2[sl, 512 + 3] = [0.0, 2.0, 1.0]
    rows2[sl, 0] = [10.0, 20.0, 30.0]  # value channel
    q = np.zeros((2, 4, 576), np.float32); q[:, :, 512 + 3] = 1.0
    scale = 1 / math.sqrt(192)
    out = oracle.mla_decode(bf(q), bf(rows2), table, lens, 4, bs, scale)
    s = np.array([0.0, 2.0, 1.0]) * scale
    p = np.exp(s - s.max()); p /= p.sum()
    assert abs(out[0, 1, 0] - (p * [10, 20, 30]).sum()) < 1e-4


def test_mla_c8_equals_bf16_on_exact_values():
    rng = np.random.default_rng(7)
    bs = 64
    lens = np.array([50, 64], np.int32)
    table = W.block_tables_for(rng, lens, bs, 2, 1)
    codes = rng.integers(-127, 128, size=(2 * bs, 512)).astype(np.int8)
    rope = W.bf16_randn(rng, (2 * bs, 64))
    packed = np.zeros((2 * bs, 656), np.uint8)
    packed[:, :512] = codes.view(np.uint8)
    packed[:, 512:640] = rope.view(np.uint8).reshape(2 * bs, 128)
    tiles = np.array([1 / 128, 1 / 64, 1 / 256, 1 / 32], np.float32)
    packed[:, 640:656] = np.tile(tiles, (2 * bs, 1)).view(np.uint8)
    deq = np.concatenate([bf(codes.astype(f32) * np.repeat(tiles, 128)[None, :]), rope], axis=1)
    q = W.bf16_randn(rng, (2, 3, 576))
    a = oracle.mla_decode(q, packed, table, lens, 3, bs, 0.07, c8=True)
    b = oracle.mla_decode(q, deq, table, lens, 3, bs, 0.07)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def test_sequence_attention_probe_known_answer():
    # native/probes/sequence_attention_probe.cpp:26-27,100 (without its 128 zero
    # sinks): q = 0, code v(slot, pos) = ((slot*31 + pos*7) % 101) - 50 in every
    # latent dim, scale 1/128 -> each output = sum_i v(slot, i)/128 / count.
    bs, slot, count = 32, 2, 70
    rng = np.random.default_rng(8)
    lens = np.array([count], np.int32)
    table = W.block_tables_for(rng, lens, bs, 4, 3)
    packed = np.zeros((4 * bs, 656), np.uint8)
    sl = _visible_slots(table, 0, count, bs)
    for pos, s in enumerate(sl):
        packed[s, :512] = np.int8((slot * 31 + pos * 7) % 101 - 50).view(np.uint8)
        packed[s, 640:656] = np.full(4, 1 / 128, np.float32).view(np.uint8)
    out = oracle.mla_decode(np.zeros((1, 6, 576), np.uint16), packed, table, lens, 6, bs,
                            1 / math.sqrt(192), c8=True)
    exp = sum(((slot * 31 + i * 7) % 101 - 50) / 128 for i in range(count)) / count
    np.testing.assert_allclose(out, exp, rtol=1e-5)
