"""GPU parity for the Qwen-shape gated attention (ifattn_gated_paged_attention_bf16,
the operation of inferfabric_acl_paged_attention_prepare,
native/src/inferfabric_acl.cpp:1343-1430) against oracle_gated_attention:
appended rows bit-exact, outputs within 1e-2 abs + 1e-2 rel and relative L2."""
import numpy as np
import pytest

import oracle
from helpers import assert_close, assert_rel_l2, bf16_host, bits_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu

HQ, HKV, D = 8, 2, 256


def _run(seed, batch, context, slots, holes=0.0, finite_mask=False):
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, context + 1, batch)
    lens[0] = context
    # every position of every request gets its own physical row (random order);
    # the step's new row is the request's last live position
    rows = rng.permutation(slots)[: batch * context].reshape(batch, context).astype(np.int64)
    pos = np.arange(context)
    live = pos[None, :] < lens[:, None]
    if holes:
        live &= ~((rng.random((batch, context)) < holes) & (pos[None, :] < lens[:, None] - 1))
    mask = np.where(live, 0.0, -np.inf).astype(np.float32)
    if finite_mask:  # finite additive biases on live positions
        mask = np.where(live, rng.uniform(-4, 1, (batch, context)), -np.inf).astype(np.float32)
    append = rows[np.arange(batch), lens - 1].copy()
    _check(rng, rows, mask, append, slots)


def _check(rng, rows, mask, append, slots):
    """Run the operator on random caches/q/k/v/gate and compare with the oracle."""
    import torch
    from ironpangu_amd import ops
    batch = rows.shape[0]
    keys = W.bf16_randn(rng, (slots, HKV * D))
    values = W.bf16_randn(rng, (slots, HKV * D))
    q = W.bf16_randn(rng, (batch, HQ, D))
    k = W.bf16_randn(rng, (batch, HKV * D))
    v = W.bf16_randn(rng, (batch, HKV * D))
    gate = W.bf16_bits(1.0 / (1.0 + np.exp(-rng.standard_normal((batch, HQ, D)).astype(np.float32))))
    kd, vd = to_dev(keys), to_dev(values)
    out = ops.gated_paged_attention(to_dev(q), to_dev(k), to_dev(v), to_dev(gate), kd, vd,
                                    to_dev(append), to_dev(rows), to_dev(mask))
    torch.cuda.synchronize()
    oracle.kv_write(k, keys, append)
    oracle.kv_write(v, values, append)
    assert np.array_equal(bits_host(kd), keys), "appended K rows not bit-exact"
    assert np.array_equal(bits_host(vd), values), "appended V rows not bit-exact"
    exp = oracle.gated_attention(q, keys, values, rows, mask, gate, threads=16)
    got = bf16_host(out)
    assert_rel_l2(got, exp, what="gated attention")
    assert_close(got, exp, what="gated attention")


# Partition lengths follow (batch, context): 64 positions for these small
# calls (one partition for context <= 64), 256 for the ragged batch below.
@pytest.mark.parametrize("batch,context,holes,finite", [(3, 50, 0.0, False),      # one partition
                                                        (3, 700, 0.0, False),     # 11 partitions
                                                        (7, 3000, 0.0, False),
                                                        (5, 2500, 0.3, True),     # holes + biases
                                                        (64, 129, 0.5, False)])   # batch 64
def test_gated_attention(batch, context, holes, finite):
    _run(batch * 1000 + context, batch, context, batch * context + 17, holes, finite)


def test_gated_attention_ragged_batch_256_position_partitions():
    # 16 requests over a 32768-position table, live lengths log-uniform
    # [128, 32768] (the benchmark's shape at a quarter of its batch): 256-position
    # partitions, most of them without a live position. Rows drawn from a
    # 65536-row pool (repeats allowed); the appended rows are distinct rows
    # outside it.
    rng = np.random.default_rng(77)
    batch, context, pool = 16, 32768, 65536
    lens = W.lengths(rng, batch, 128, context, "loguniform")
    lens[0] = context
    rows = rng.integers(0, pool, (batch, context)).astype(np.int64)
    append = pool + np.arange(batch, dtype=np.int64)
    rows[np.arange(batch), lens - 1] = append
    mask = np.where(np.arange(context)[None, :] < lens[:, None], 0.0, -np.inf).astype(np.float32)
    _check(rng, rows, mask, append, pool + batch)


def test_gated_attention_live_positions_after_dead_partitions():
    # live windows that start deep in the table: whole leading partitions have
    # no live position, and one request's only live positions are its last 3
    rng = np.random.default_rng(78)
    batch, context = 4, 9000
    slots = batch * context + 5
    rows = rng.permutation(slots)[: batch * context].reshape(batch, context).astype(np.int64)
    pos = np.arange(context)
    starts = np.array([5000, 64, 8997, 1234])
    ends = np.array([9000, 300, 9000, 7000])
    live = (pos[None, :] >= starts[:, None]) & (pos[None, :] < ends[:, None])
    mask = np.where(live, 0.0, -np.inf).astype(np.float32)
    append = rows[np.arange(batch), ends - 1].copy()
    _check(rng, rows, mask, append, slots)


@pytest.mark.parametrize("context", [100, 1100])
def test_gated_attention_plan_chunk_edges(context):
    """The plan lists each request's live partitions in four chunks of
    ceil(parts / 4) partitions (two 64-position partitions at context 100:
    chunks 2 and 3 empty; 18 at 1100: chunks of 5, 5, 5, 3). Live positions sit
    only on the first and last position of chunks, and one request's only live
    positions are in its last chunk."""
    rng = np.random.default_rng(context)
    batch = 5
    slots = batch * context + 9
    rows = rng.permutation(slots)[: batch * context].reshape(batch, context).astype(np.int64)
    parts = (context + 63) // 64
    pc = (parts + 3) // 4
    edges = sorted({min(c * pc * 64, context - 1) for c in range(5)} |
                   {min((c + 1) * pc * 64 - 1, context - 1) for c in range(4)})
    live = np.zeros((batch, context), bool)
    live[0, edges] = True
    live[1, -1] = True                      # only the last position
    live[2, :] = True
    live[3, ::97] = True
    live[4, min(3 * pc * 64, context - 1):] = True  # the last chunk only
    mask = np.where(live, 0.0, -np.inf).astype(np.float32)
    last = np.array([np.nonzero(r)[0][-1] for r in live])
    append = rows[np.arange(batch), last].copy()
    _check(rng, rows, mask, append, slots)


def test_gated_attention_long_context():
    # 4 requests over 65536 positions (512 partitions of 128, merged), 2^18 + 3 slots
    _run(42, 4, 65536, (1 << 18) + 3)


def test_gated_attention_bench_size():
    """The bench's gated workload at its size: 64 requests over a
    32768-position table, live lengths log-uniform [128, 32768] (mask -inf
    beyond), rows drawn at random, with repeats, from a 2^20-row pool."""
    print("gated bench size", flush=True)
    rng = np.random.default_rng(77)
    batch, context, slots = 64, 32768, 1 << 20
    lens = W.lengths(rng, batch, 128, context, "loguniform")
    rows = rng.integers(0, slots, (batch, context)).astype(np.int64)
    mask = np.where(np.arange(context)[None, :] < lens[:, None], 0.0, -np.inf).astype(np.float32)
    append = rows[np.arange(batch), lens - 1].copy()
    _check(rng, rows, mask, append, slots)


def test_gated_attention_all_masked_request_is_zero():
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(5)
    batch, context, slots = 2, 1500, 4000
    keys = to_dev(W.bf16_randn(rng, (slots, 512)))
    values = to_dev(W.bf16_randn(rng, (slots, 512)))
    q = to_dev(W.bf16_randn(rng, (batch, 8, 256)))
    kv = to_dev(W.bf16_randn(rng, (batch, 512)))
    gate = to_dev(W.bf16_bits(np.ones((batch, 8, 256), np.float32)))
    rows = to_dev(rng.integers(0, slots, (batch, context)).astype(np.int64))
    mask = np.zeros((batch, context), np.float32)
    mask[1] = -np.inf
    out = ops.gated_paged_attention(q, kv, kv, gate, keys, values,
                                    to_dev(np.array([0, 1], np.int64)), rows, to_dev(mask))
    torch.cuda.synchronize()
    o = bf16_host(out)
    assert np.all(o[1] == 0) and np.isfinite(o).all() and np.abs(o[0]).sum() > 0


def test_gated_attention_rejects_limits():
    import torch
    from ironpangu_amd._native import IfattnError
    from ironpangu_amd import ops
    z = lambda *s, dt=torch.bfloat16: torch.zeros(*s, dtype=dt, device="cuda")
    with pytest.raises(IfattnError):  # batch 65 > 64
        ops.gated_paged_attention(z(65, 8, 256), z(65, 512), z(65, 512), z(65, 8, 256), z(8, 512),
                                  z(8, 512), z(65, dt=torch.int64), z(65, 4, dt=torch.int64),
                                  z(65, 4, dt=torch.float32))
