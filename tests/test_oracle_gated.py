"""Pins for oracle_gated_attention, the CPU restatement of the Qwen-shape
session attention (native/src/inferfabric_acl.cpp:1343-1430): scatter, gather
by per-position rows, scores * 1/16 + fp32 additive mask, softmax, PV, gate.

Each check is chosen so a plausible mistake fails it: a mask that opens a
prefix must reproduce the independently pinned paged decode (wrong grouping,
scale or gather), a constant mask shift must not change anything (mask added
after the softmax or in the wrong units), the gate must act linearly per
element (gate applied before normalisation or on the wrong axis), and a
two-position closed form fixes the sign and scale of mask and score."""
import math

import numpy as np

import oracle
from ironpangu_amd import workloads as W

HQ, HKV, D = 8, 2, 256


def bf(x):
    return W.bf16_bits(np.asarray(x, np.float32))


def _case(seed, batch=5, context=300, bs=32):
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, context + 1, batch).astype(np.int32)
    pool = int(((lens + bs - 1) // bs).sum()) + 2
    tables = W.block_tables_for(rng, lens, bs, pool, (context + bs - 1) // bs)
    keys = W.bf16_randn(rng, (pool * bs, HKV * D))
    values = W.bf16_randn(rng, (pool * bs, HKV * D))
    q = W.bf16_randn(rng, (batch, HQ, D))
    pos = np.arange(context)
    rows = (tables[:, pos // bs].astype(np.int64) * bs + pos % bs)
    mask = np.where(pos[None, :] < lens[:, None], 0.0, -np.inf).astype(np.float32)
    rows = np.where(pos[None, :] < lens[:, None], rows, 0)
    return rng, lens, tables, keys, values, q, rows, mask


def test_open_prefix_equals_paged_decode():
    _, lens, tables, keys, values, q, rows, mask = _case(1)
    gate = np.full(q.shape, bf(1.0), np.uint16)
    got = oracle.gated_attention(q, keys, values, rows, mask, gate)
    exp = oracle.paged_decode(q, keys, values, tables, lens, HQ, HKV, D, 32, 0.0625)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)


def test_mask_shift_invariance_and_gate_linearity():
    rng, lens, tables, keys, values, q, rows, mask = _case(2)
    gate = W.bf16_randn(rng, q.shape)
    base = oracle.gated_attention(q, keys, values, rows, mask, gate)
    shifted = oracle.gated_attention(q, keys, values, rows, mask + np.float32(3.0), gate)
    np.testing.assert_allclose(shifted, base, rtol=1e-5, atol=1e-6)
    # gate doubles exactly (a power of two) and acts per element
    g2 = bf(W.bf16_to_f32(gate) * 2.0)
    np.testing.assert_array_equal(oracle.gated_attention(q, keys, values, rows, mask, g2), 2 * base)
    ones = np.full(q.shape, bf(1.0), np.uint16)
    ungated = oracle.gated_attention(q, keys, values, rows, mask, ones)
    np.testing.assert_allclose(base, ungated * W.bf16_to_f32(gate), rtol=1e-6, atol=1e-7)


def test_two_position_closed_form():
    # head 5 reads kv head 1; its q is 8 on dim 0. Row 0 of kv head 1 has K = 1 on
    # dim 0 and V = 1; row 1 has K = 0 and V = 3. Scores 0.5 and 0, masks 0 and
    # 0.25: p0 = 1 / (1 + exp(0.25 - 0.5)).
    keys = np.zeros((2, HKV * D), np.uint16)
    values = np.zeros((2, HKV * D), np.uint16)
    keys[0, D] = bf(1.0)
    values[0, D:] = bf(1.0)
    values[1, D:] = bf(3.0)
    values[:, :D] = bf(7.0)  # kv head 0: must not leak into head 5
    q = np.zeros((1, HQ, D), np.uint16)
    q[0, 5, 0] = bf(8.0)
    table = np.array([[0, 1]], np.int64)
    mask = np.array([[0.0, 0.25]], np.float32)
    gate = np.full(q.shape, bf(0.5), np.uint16)
    out = oracle.gated_attention(q, keys, values, table, mask, gate)
    p0 = 1.0 / (1.0 + math.exp(0.25 - 0.5))
    np.testing.assert_allclose(out[0, 5], 0.5 * (p0 * 1 + (1 - p0) * 3), rtol=1e-6)
    np.testing.assert_allclose(out[0, 0], 0.5 * 7.0, rtol=1e-6)  # kv head 0: V = 7 everywhere
    # all positions masked: defined zero output
    dead = oracle.gated_attention(q, keys, values, table, np.full((1, 2), -np.inf, np.float32), gate)
    assert np.all(dead == 0)
