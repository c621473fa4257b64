"""GPU parity: slot-mapped KV write (bit-exact) and ragged paged GQA decode
(bf16 output within 1e-2 abs/rel of the fp32 oracle) through the C ABI."""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_close, bf16_host, bits_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _step(case, max_context=None):
    """Upload the pools, run write + decode on the GPU and on the oracle."""
    import torch
    from ironpangu_amd import ops
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    slots = to_dev(case.slot_mapping.astype(np.int64))
    ops.kv_cache_write(to_dev(h["k_new"]), to_dev(h["v_new"]), kc, vc, slots)
    out = ops.paged_decode(to_dev(h["q"]), kc, vc, to_dev(case.block_tables),
                           to_dev(case.seq_lens), max_context or case.max_context, case.scale)
    torch.cuda.synchronize()
    k_ref, v_ref = h["k_pool"].copy(), h["v_pool"].copy()
    oracle.kv_write(h["k_new"], k_ref, case.slot_mapping)
    oracle.kv_write(h["v_new"], v_ref, case.slot_mapping)
    exp = oracle.paged_decode(h["q"], k_ref, v_ref, case.block_tables, case.seq_lens,
                              case.q_heads, hkv, hd, bs, case.scale)
    return kc, vc, k_ref, v_ref, out, exp


def test_config1_write_and_decode():
    case = W.config_case("cpu_ref", seed=1)
    kc, vc, k_ref, v_ref, out, exp = _step(case)
    assert np.array_equal(bits_host(kc).reshape(k_ref.shape), k_ref), "K cache not bit-exact"
    assert np.array_equal(bits_host(vc).reshape(v_ref.shape), v_ref), "V cache not bit-exact"
    assert_close(bf16_host(out), exp)


@pytest.mark.parametrize("hq,hkv,hd,bs", [(16, 2, 128, 128), (16, 2, 128, 32), (8, 2, 256, 64),
                                          (8, 8, 64, 32), (32, 2, 128, 64)])
def test_decode_shapes(hq, hkv, hd, bs):
    case = W.decode_host_case(7, num_seqs=6, lo=1, hi=1100, dist="uniform", q_heads=hq,
                              kv_heads=hkv, head_dim=hd, block_size=bs,
                              pool_blocks=6 * ((1100 + bs - 1) // bs) + 3)
    case.seq_lens[:4] = [1, 256, 257, 1100][:4]
    # keep the slot mapping consistent with the edited lengths
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(6), bs)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)


def test_decode_head_dim_256_split_k():
    # head_dim 256 (two-stage register ring) over several split-K partitions
    lens = [1, 33, 2047, 2048, 2049, 6000]
    case = W.decode_host_case(11, num_seqs=len(lens), lo=1, hi=6000, dist="uniform", q_heads=8,
                              kv_heads=2, head_dim=256, block_size=128, pool_blocks=300)
    case.seq_lens[:] = lens
    case.block_tables = W.block_tables_for(np.random.default_rng(6), case.seq_lens, 128, 300,
                                           case.block_tables.shape[1])
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(len(lens)), 128)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)


def test_decode_many_partitions():
    # more than 16 split-K partitions per sequence: the merge's multi-round path
    lens = [1, 40000, 70001]
    case = W.decode_host_case(13, num_seqs=len(lens), lo=1, hi=70001, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=128, pool_blocks=1800)
    case.seq_lens[:] = lens
    case.block_tables = W.block_tables_for(np.random.default_rng(8), case.seq_lens, 128, 1800,
                                           case.block_tables.shape[1])
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(len(lens)), 128)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)


def test_decode_shares_slide_the_block_window():
    # 16-token pages hold 128 block ids per lane window (2048 tokens); two
    # 600000-token sequences give each of the persistent workgroups a share of
    # about 2350 tokens, so the window slides inside a share, and each
    # sequence spreads over about 256 shares (many merge rounds).
    lens = [600000, 599991]
    bs, nb = 16, 2 * 37500 + 64
    case = W.decode_host_case(19, num_seqs=len(lens), lo=1, hi=600000, dist="uniform", q_heads=8,
                              kv_heads=1, head_dim=64, block_size=bs, pool_blocks=nb)
    case.seq_lens[:] = lens
    case.block_tables = W.block_tables_for(np.random.default_rng(9), case.seq_lens, bs, nb,
                                           case.block_tables.shape[1])
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(len(lens)), bs)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)


def test_decode_many_sequences():
    # a large ragged batch of short sequences (more items than workgroups, and
    # sequence ids beyond 4096 in the work-item encoding)
    case = W.decode_host_case(17, num_seqs=5000, lo=1, hi=300, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=32, pool_blocks=5000 * 10 + 8)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)


def test_decode_partition_edges_and_long():
    # lengths around the 2048-token split-K partition and 32-token tile edges
    lens = [31, 32, 33, 255, 256, 257, 511, 512, 513, 4095, 8193]
    case = W.decode_host_case(3, num_seqs=len(lens), lo=1, hi=8193, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=128, pool_blocks=720)
    case.seq_lens[:] = lens
    case.block_tables = W.block_tables_for(np.random.default_rng(5), case.seq_lens, 128, 720,
                                           case.block_tables.shape[1])
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(len(lens)), 128)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)


def test_decode_zero_length_gives_zero():
    import torch
    from ironpangu_amd import ops
    case = W.decode_host_case(11, num_seqs=3, lo=5, hi=40, dist="uniform", q_heads=16, kv_heads=2,
                              head_dim=128, block_size=32, pool_blocks=8)
    lens = case.seq_lens.copy()
    lens[1] = 0
    h = case.host
    kc = to_dev(h["k_pool"]).view(8, 32, 2, 128)
    vc = to_dev(h["v_pool"]).view(8, 32, 2, 128)
    out = ops.paged_decode(to_dev(h["q"]), kc, vc, to_dev(case.block_tables), to_dev(lens), 40)
    torch.cuda.synchronize()
    o = bf16_host(out)
    assert np.all(o[1] == 0)
    exp = oracle.paged_decode(h["q"], h["k_pool"], h["v_pool"], case.block_tables, lens, 16, 2,
                              128, 32, case.scale)
    assert_close(o, exp)


def test_decode_rejects_bad_contracts():
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd._native import IfattnError
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(4, 8, 2, 128, dtype=torch.bfloat16, device="cuda")  # block 8 unsupported
    bt = torch.zeros(2, 8, dtype=torch.int32, device="cuda")
    sl = torch.ones(2, dtype=torch.int32, device="cuda")
    with pytest.raises(IfattnError):
        ops.paged_decode(q, kc, kc, bt, sl, 64)


@pytest.mark.parametrize("hd,c8", [(128, False), (64, False), (256, False), (128, True),
                                   (256, True)])
def test_decode_16_token_pages(hd, c8):
    """The reference's bf16 page of 16 tokens (native/include/paged_state_contract.h:25):
    32-token tiles span two pages and a 2048-token partition spans 128 pages.
    Lengths cross page, tile and partition edges; partitions run past 64 pages."""
    import torch
    from ironpangu_amd import ops
    lens = [1, 15, 16, 17, 31, 33, 1023, 1025, 2047, 2049, 5000]
    bs, pool = 16, len(lens) * ((5000 + 15) // 16) + 7  # covers the drawn lengths too
    case = W.decode_host_case(77 + hd, num_seqs=len(lens), lo=1, hi=5000, dist="uniform",
                              q_heads=8, kv_heads=2, head_dim=hd, block_size=bs, pool_blocks=pool,
                              c8=c8)
    case.seq_lens[:] = lens
    case.block_tables = W.block_tables_for(np.random.default_rng(hd), case.seq_lens, bs, pool,
                                           case.block_tables.shape[1])
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(len(lens)), bs)
    if not c8:
        *_, out, exp = _step(case)
        assert_close(bf16_host(out), exp)
        return
    h = case.host
    kc = torch.zeros((pool, bs, 2, hd), dtype=torch.int8, device="cuda")
    vc = torch.zeros_like(kc)
    ks = torch.zeros((pool, bs, 2), dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    ops.kv_cache_write_c8(to_dev(h["k_pool"]), to_dev(h["v_pool"]), kc, vc, ks, vs,
                          torch.arange(pool * bs, dtype=torch.int64, device="cuda"))
    out = ops.paged_decode(to_dev(h["q"]), kc, vc, to_dev(case.block_tables),
                           to_dev(case.seq_lens), case.max_context, case.scale, k_scale=ks,
                           v_scale=vs)
    torch.cuda.synchronize()
    exp = oracle.paged_decode(h["q"], kc.cpu().numpy(), vc.cpu().numpy(), case.block_tables,
                              case.seq_lens, 8, 2, hd, bs, case.scale, k_scale=ks.cpu().numpy(),
                              v_scale=vs.cpu().numpy())
    assert_close(bf16_host(out), exp)


def test_graph_replay_matches_eager():
    """Write + decode captured once into a HIP graph: every replay (with eager
    work and synchronisation in between) reproduces the eager result bit for bit."""
    import torch
    from ironpangu_amd import ops
    case = W.config_case("cpu_ref", seed=4)
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    k_new, v_new, q = to_dev(h["k_new"]), to_dev(h["v_new"]), to_dev(h["q"])
    slots = to_dev(case.slot_mapping.astype(np.int64))
    tables, lens = to_dev(case.block_tables), to_dev(case.seq_lens)
    ws = ops.decode_workspace(case.num_seqs, case.q_heads, hd, case.max_context)
    out = torch.empty_like(q)

    def step():
        ops.kv_cache_write(k_new, v_new, kc, vc, slots)
        ops.paged_decode(q, kc, vc, tables, lens, case.max_context, case.scale, out=out,
                         workspace=ws)

    step()
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(3):
        out.fill_(0)
        ws.fill_(255)  # scheduling words must be rebuilt by the replay itself
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"


def test_decode_step_matches_write_then_decode():
    """The fused step (write folded into the decode prologue) equals a separate
    write followed by decode, bit for bit, including partitioned sequences."""
    import torch
    from ironpangu_amd import ops
    case = W.decode_host_case(12, num_seqs=9, lo=1, hi=9000, dist="loguniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=128, pool_blocks=9 * 71)
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc1 = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc1 = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    kc2, vc2 = kc1.clone(), vc1.clone()
    args = (to_dev(h["q"]), to_dev(h["k_new"]), to_dev(h["v_new"]))
    slots = to_dev(case.slot_mapping.astype(np.int32))
    tables, lens = to_dev(case.block_tables), to_dev(case.seq_lens)
    out1 = ops.paged_decode_step(args[0], args[1], args[2], kc1, vc1, slots, tables, lens,
                                 case.max_context, case.scale)
    ops.kv_cache_write(args[1], args[2], kc2, vc2, slots)
    out2 = ops.paged_decode(args[0], kc2, vc2, tables, lens, case.max_context, case.scale)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(out1, out2)
    exp = oracle.paged_decode(h["q"], bits_host(kc2).reshape(-1, hkv, hd),
                              bits_host(vc2).reshape(-1, hkv, hd), case.block_tables,
                              case.seq_lens, 16, 2, 128, 128, case.scale)
    assert_close(bf16_host(out1), exp)


@pytest.mark.parametrize("seed", range(12))
def test_decode_random_shapes(seed):
    """Seeded random shapes across the K/V load paths (whole-line bf16 K loads
    with lane rotation at head_dim 64/128/256, 16- and 32-token tiles, group
    sizes 1..16, block sizes 16..128) with ragged lengths that cross tile,
    block and split-K partition edges."""
    rng = np.random.default_rng(1000 + seed)
    hd = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([g for g in (1, 2, 4, 8, 16) if g * hkv <= 64]))
    bs = int(rng.choice([16, 32, 64, 128]))
    n = int(rng.integers(1, 12))
    hi = int(rng.choice([40, 700, 2500, 5000]))
    lens = rng.integers(1, hi + 1, n)
    lens[0] = hi
    need = n * ((hi + bs - 1) // bs)  # covers the lengths decode_meta draws and these
    case = W.decode_host_case(2000 + seed, num_seqs=n, lo=1, hi=hi, dist="uniform",
                              q_heads=group * hkv, kv_heads=hkv, head_dim=hd, block_size=bs,
                              pool_blocks=need + 4)
    case.seq_lens[:] = lens
    case.block_tables = W.block_tables_for(np.random.default_rng(seed), case.seq_lens, bs, need + 4,
                                           case.block_tables.shape[1])
    case.slot_mapping = W.slots_of(case.block_tables, case.seq_lens - 1, np.arange(n), bs)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp, what=f"hd {hd} hkv {hkv} group {group} bs {bs} lens {list(lens)}")


@pytest.mark.parametrize("hkv,num_seqs", [(1, 256), (1, 257), (2, 512), (2, 513)])
def test_decode_self_plan_limit(hkv, num_seqs):
    # calls of up to four sequences per decode thread (one wave per kv head)
    # plan inside the decode workgroups; one more sequence takes the prologue's
    # plan; zero-length sequences and sequences over several shares included
    case = W.decode_host_case(41 + num_seqs, num_seqs=num_seqs, lo=1, hi=3000, dist="loguniform",
                              q_heads=8 * hkv, kv_heads=hkv, head_dim=128, block_size=64,
                              pool_blocks=num_seqs * (3000 // 64 + 1) + 4)
    case.seq_lens[::53] = 0
    case.seq_lens[7::61] = 3000
    case.block_tables = W.block_tables_for(np.random.default_rng(num_seqs), case.seq_lens, 64,
                                           case.pool_blocks, case.block_tables.shape[1])
    live = np.nonzero(case.seq_lens > 0)[0]
    case.slot_mapping = np.full(num_seqs, -1, np.int64)
    case.slot_mapping[live] = W.slots_of(case.block_tables[live], case.seq_lens[live] - 1,
                                         np.arange(len(live)), 64)
    *_, out, exp = _step(case)
    assert_close(bf16_host(out), exp)
