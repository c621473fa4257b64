"""GPU parity at the benchmark's full sizes (and config 5 over row-quantized rows), on the same
seeded metadata bench.py times (seed 0 of ironpangu_amd.workloads).

Each test builds the whole pool on the GPU, runs the HIP path through the C
ABI, and checks it against the CPU oracle:
  * cache writes bit-exact over the WHOLE pool (the written rows hold the new
    rows, every other row is unchanged), int8 codes and scales bit-exact;
  * attention outputs within 1e-2 abs + 1e-2 rel of the fp32 oracle, which
    runs on a compact host copy of exactly the blocks the batch references
    (tables remapped onto it), so host memory stays bounded.
The untouched-row rule follows native/probes/prefill_cache_writer_probe.cpp:36-37;
the attention math is crates/inferfabric-cli/src/npu_probe/attention.rs:221-253.
"""
import numpy as np
import pytest

import oracle
from helpers import (assert_close, assert_rel_l2, bf16_host, bits_host, compact_blocks, fill_randn, remap_slots,
                     to_dev)
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu

THREADS = 16  # the box's CPU share for one GPU


def _gen(seed):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def _randn(g, shape, std=1.0, clip=None):
    import torch
    x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * std
    if clip is not None:
        x.clamp_(-clip, clip)
    return x.to(torch.bfloat16)


def _gather_host(pool, used):
    """Blocks `used` of a device pool [blocks, ...] -> numpy (bf16 as uint16 bits)."""
    import torch
    sel = pool.index_select(0, torch.from_numpy(used).to(pool.device))
    if sel.dtype == torch.bfloat16:
        return bits_host(sel)
    return sel.cpu().numpy()


def _check_rows_written_rest_unchanged(pool, before, slots_d, new_rows):
    """Whole-pool write check on the device: rows at `slots_d` equal `new_rows`
    bit for bit, and every other row equals the pre-write clone. The clone
    `before` is overwritten (it becomes the expected pool); `pool` is not."""
    import torch
    flat = pool.view(pool.shape[0] * pool.shape[1], -1)
    assert torch.equal(flat.index_select(0, slots_d).view(torch.uint8),
                       new_rows.reshape(new_rows.shape[0], -1).view(torch.uint8)), \
        "written rows differ from the new rows"
    before.view(flat.shape).index_copy_(0, slots_d, flat.index_select(0, slots_d))
    assert torch.equal(pool.view(torch.uint8), before.view(torch.uint8)), \
        "a row outside the slot mapping changed"


def test_config2_decode_step_full_size():
    """Config 2: 256 seqs, log-uniform [128, 32768], 65536-block pool; the
    fused step (slot write of 256 K/V rows + ragged decode)."""
    import torch
    from ironpangu_amd import ops
    case = W.decode_meta(0, **W.CONFIGS["decode"])
    nb, bs, hkv, hd, hq = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim, case.q_heads
    print(f"config2: {case.num_seqs} seqs, {int(case.seq_lens.sum())} tokens", flush=True)
    g = _gen(200)
    kc = torch.empty((nb, bs, hkv, hd), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    fill_randn(kc, g)
    fill_randn(vc, g)
    q = _randn(g, (case.num_seqs, hq, hd))
    kn = _randn(g, (case.num_seqs, hkv, hd))
    vn = _randn(g, (case.num_seqs, hkv, hd))
    used, ctab = compact_blocks(case.block_tables, case.seq_lens, bs)
    k_ref, v_ref = _gather_host(kc, used), _gather_host(vc, used)
    k_before, v_before = kc.clone(), vc.clone()
    slots_d = to_dev(case.slot_mapping.astype(np.int64))
    out = ops.paged_decode_step(q, kn, vn, kc, vc, slots_d, to_dev(case.block_tables),
                                to_dev(case.seq_lens), case.max_context, case.scale)
    torch.cuda.synchronize()
    _check_rows_written_rest_unchanged(kc, k_before, slots_d, kn)
    _check_rows_written_rest_unchanged(vc, v_before, slots_d, vn)
    del k_before, v_before
    cslots = remap_slots(case.slot_mapping, used, bs)
    oracle.kv_write(bits_host(kn), k_ref, cslots)
    oracle.kv_write(bits_host(vn), v_ref, cslots)
    exp = oracle.paged_decode(bits_host(q), k_ref, v_ref, ctab, case.seq_lens, hq, hkv, hd, bs,
                              case.scale, threads=THREADS)
    assert_rel_l2(bf16_host(out), exp, what="config-2 decode")
    assert_close(bf16_host(out), exp, what="config-2 decode")


def test_config4_c8_decode_full_size():
    """Config 4: C8 pool quantized by the C8 write from N(0,1) clipped to +-4
    (round half even, fp32 scale per token per kv head); 256 seqs U[1024, 16384]."""
    import torch
    from ironpangu_amd import ops
    case = W.decode_meta(0, c8=True, **W.CONFIGS["c8"])
    nb, bs, hkv, hd, hq = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim, case.q_heads
    print(f"config4: {case.num_seqs} seqs, {int(case.seq_lens.sum())} tokens", flush=True)
    g = _gen(400)
    kc = torch.empty((nb, bs, hkv, hd), dtype=torch.int8, device="cuda")
    vc = torch.empty_like(kc)
    ks = torch.empty((nb, bs, hkv), dtype=torch.float32, device="cuda")
    vs = torch.empty_like(ks)
    rows = 1 << 18
    for r0 in range(0, nb * bs, rows):
        sk = _randn(g, (rows, hkv, hd), clip=4.0)
        sv = _randn(g, (rows, hkv, hd), clip=4.0)
        ops.kv_cache_write_c8(sk, sv, kc, vc, ks, vs,
                              torch.arange(r0, r0 + rows, dtype=torch.int64, device="cuda"))
        if r0 == 0:  # one slab of pool rows checked bit-exact against the oracle
            torch.cuda.synchronize()
            codes, scales = oracle.quant_rows(bits_host(sk), hd)
            got = kc.view(-1, hd)[: rows * hkv].cpu().numpy()
            assert np.array_equal(got, codes), "pool codes differ"
            assert np.array_equal(ks.view(-1)[: rows * hkv].cpu().numpy(), scales), "pool scales differ"
    q = _randn(g, (case.num_seqs, hq, hd))
    kn = _randn(g, (case.num_seqs, hkv, hd), clip=4.0)
    vn = _randn(g, (case.num_seqs, hkv, hd), clip=4.0)
    slots_d = to_dev(case.slot_mapping.astype(np.int64))
    before = [t.clone() for t in (kc, vc, ks, vs)]
    ops.kv_cache_write_c8(kn, vn, kc, vc, ks, vs, slots_d)
    out = ops.paged_decode(q, kc, vc, to_dev(case.block_tables), to_dev(case.seq_lens),
                           case.max_context, case.scale, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    for new, pool, scl, b_pool, b_scl in ((kn, kc, ks, before[0], before[2]),
                                          (vn, vc, vs, before[1], before[3])):
        codes, scales = oracle.quant_rows(bits_host(new), hd)
        ccodes = torch.from_numpy(codes.reshape(case.num_seqs, hkv, hd)).cuda()
        cscales = torch.from_numpy(scales.reshape(case.num_seqs, hkv)).cuda()
        _check_rows_written_rest_unchanged(pool, b_pool, slots_d, ccodes)
        _check_rows_written_rest_unchanged(scl, b_scl, slots_d, cscales)
    del before
    used, ctab = compact_blocks(case.block_tables, case.seq_lens, bs)
    exp = oracle.paged_decode(bits_host(q), _gather_host(kc, used), _gather_host(vc, used), ctab,
                              case.seq_lens, hq, hkv, hd, bs, case.scale,
                              k_scale=_gather_host(ks, used), v_scale=_gather_host(vs, used),
                              threads=THREADS)
    assert_rel_l2(bf16_host(out), exp, what="config-4 C8 decode")
    assert_close(bf16_host(out), exp, what="config-4 C8 decode")


@pytest.mark.parametrize("c8", [False, True], ids=["bf16", "c8"])
def test_config5_mla_decode_full_size(c8):
    """Config 5: 128 seqs, log-uniform [1024, 65536], 16 heads, 576-wide rows,
    block 64, N(0, 0.5); bf16 rows (1152 B) or packed C8 rows (656 B)."""
    import torch
    from ironpangu_amd import ops
    case = W.mla_meta(0)
    nb, bs, heads = case.pool_blocks, case.block_size, case.heads
    print(f"config5 {'c8' if c8 else 'bf16'}: {case.num_seqs} seqs, "
          f"{int(case.seq_lens.sum())} tokens", flush=True)
    g = _gen(500 + int(c8))
    slots_d = to_dev(case.slot_mapping.astype(np.int64))
    if c8:
        cache = torch.empty((nb, bs, 656), dtype=torch.uint8, device="cuda")
        rows = 1 << 16
        for r0 in range(0, nb * bs, rows):
            m = min(rows, nb * bs - r0)
            src = _randn(g, (m, 576), std=0.5)
            ops.mla_cache_write_c8(src, cache, torch.arange(r0, r0 + m, dtype=torch.int64,
                                                            device="cuda"))
            if r0 == 0:
                torch.cuda.synchronize()
                assert np.array_equal(cache.view(-1, 656)[:m].cpu().numpy(),
                                      oracle.mla_pack_c8(bits_host(src))), "packed pool rows differ"
    else:
        cache = torch.empty((nb, bs, 576), dtype=torch.bfloat16, device="cuda")
        fill_randn(cache, g, std=0.5)
    q = _randn(g, (case.num_seqs, heads, 576), std=0.5)
    new = _randn(g, (case.num_seqs, 576), std=0.5)
    before = cache.clone()
    if c8:
        ops.mla_cache_write_c8(new, cache, slots_d)
    else:
        ops.kv_cache_write(new, None, cache, None, slots_d)
    out = ops.mla_decode(q, cache, to_dev(case.block_tables), to_dev(case.seq_lens),
                         case.max_context, case.scale)
    torch.cuda.synchronize()
    expect_rows = torch.from_numpy(oracle.mla_pack_c8(bits_host(new))).cuda() if c8 else new
    _check_rows_written_rest_unchanged(cache, before, slots_d, expect_rows)
    del before
    used, ctab = compact_blocks(case.block_tables, case.seq_lens, bs)
    exp = oracle.mla_decode(bits_host(q), _gather_host(cache, used), ctab, case.seq_lens, heads,
                            bs, case.scale, c8=c8, threads=THREADS)
    assert_rel_l2(bf16_host(out), exp, what=f"config-5 MLA decode ({'c8' if c8 else 'bf16'})")
    assert_close(bf16_host(out), exp, what=f"config-5 MLA decode ({'c8' if c8 else 'bf16'})")


@pytest.mark.parametrize("bits", [8, 4])
def test_config5_rowq_full_size(bits):
    """Config 5's rows and lengths over row-quantized rows (int8 or int4 codes of
    all 576 dims, one fp32 scale per row; the bench's mla_decode_rowq lines):
    every row against the oracle's attention over the bf16 rows
    oracle_dequant_legacy gives for the referenced blocks (the reference's
    dequantize-then-attend path). Codes are uniform over the whole code range
    and scales vary per row, so every code value and a range of scales occur."""
    import torch
    from ironpangu_amd import ops
    case = W.mla_meta(0)
    nb, bs, heads = case.pool_blocks, case.block_size, case.heads
    row_bytes = 576 * bits // 8
    print(f"config5 rowq{bits}: {case.num_seqs} seqs, {int(case.seq_lens.sum())} tokens", flush=True)
    g = _gen(700 + bits)
    cache = torch.randint(0, 256, (nb, bs, row_bytes), generator=g, device="cuda", dtype=torch.uint8)
    if bits == 8:
        cache[cache == 128] = 129  # -128 is outside the quantizer's [-127, 127]
    scales = torch.rand(nb * bs, generator=g, device="cuda") * 0.01 + 0.001
    q = _randn(g, (case.num_seqs, heads, 576), std=0.5)
    out = ops.mla_attention(q, cache, to_dev(case.block_tables), to_dev(case.seq_lens), case.max_context,
                            scale=case.scale, row_scales=scales, bits=bits)
    torch.cuda.synchronize()
    used, ctab = compact_blocks(case.block_tables, case.seq_lens, bs)
    codes = _gather_host(cache, used).reshape(-1)
    sc = scales.view(nb, bs).index_select(0, torch.from_numpy(used).cuda()).cpu().numpy().reshape(-1)
    del cache
    rows = sc.size
    deq = oracle.dequant_legacy(codes, sc, rows - 1, 576, bits).reshape(rows, 576)
    exp = oracle.mla_attention(bits_host(q), deq, ctab, case.seq_lens, heads, bs, case.scale,
                               threads=THREADS)
    assert_rel_l2(bf16_host(out), exp, what=f"config-5 MLA decode (rowq{bits})")
    assert_close(bf16_host(out), exp, what=f"config-5 MLA decode (rowq{bits})")


@pytest.mark.parametrize("sparse", [False, True], ids=["window2048", "sparse2048"])
def test_mla_sinks_bench_size(sparse):
    """The bench's small-call MLA workloads at their size: 128 decode rows over
    contexts U[4096, 65536], 16 heads, 128 learned sinks; bf16 rows behind a
    2048-token window on 16-token ring pages, or packed C8 rows behind random
    top-2048 causal candidate lists on 32-token pages. Every row against the
    oracle; the sparse case hands the oracle a compact pool of exactly the
    referenced rows (one row per block) with the tables remapped onto it."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd.host import WindowLayout
    rng = np.random.default_rng(41)
    n, heads, topk, window, ctx = 128, 16, 2048, 2048, 65536
    bs = 32 if sparse else 16
    lens = rng.integers(4096, 65537, n).astype(np.int32)
    print(f"mla sinks bench size sparse={sparse}", flush=True)
    if sparse:
        need = (lens.astype(np.int64) + bs - 1) // bs
        pool = int(need.sum())
        table = W.block_tables_for(rng, lens, bs, pool, ctx // bs)
    else:
        lay = WindowLayout(ctx, window, 1, bs)
        pool = n * lay.physical_pages
        table = np.stack([lay.table(np.arange(lay.physical_pages) + s * lay.physical_pages)
                          for s in range(n)]).astype(np.int32)
    g = _gen(900 + int(sparse))
    if sparse:
        cache = torch.empty((pool, bs, 656), dtype=torch.uint8, device="cuda")
        for r0 in range(0, pool * bs, 1 << 16):
            m = min(1 << 16, pool * bs - r0)
            ops.mla_cache_write_c8(_randn(g, (m, 576), std=0.5), cache,
                                   torch.arange(r0, r0 + m, dtype=torch.int64, device="cuda"))
        idx = np.stack([rng.permutation(int(lens[i]))[:topk] for i in range(n)]).astype(np.int32)
    else:
        cache = torch.empty((pool, bs, 576), dtype=torch.bfloat16, device="cuda")
        fill_randn(cache, g, std=0.5)
        idx = None
    q = _randn(g, (n, heads, 576), std=0.5)
    sk = _randn(g, (128, 576), std=0.5)
    sv = _randn(g, (128, 512), std=0.5)
    out = ops.mla_attention(q, cache, to_dev(table), to_dev(lens), ctx,
                            indices=None if idx is None else to_dev(idx),
                            window=0 if sparse else window, sink_keys=sk, sink_values=sv)
    torch.cuda.synchronize()
    if sparse:
        # physical row of every candidate, then a pool of those rows alone
        phys = table[np.arange(n)[:, None], idx // bs].astype(np.int64) * bs + idx % bs
        rows, inv = np.unique(phys, return_inverse=True)
        host = cache.view(-1, 656).index_select(0, torch.from_numpy(rows).cuda()).cpu().numpy()
        ctab = np.zeros((n, ctx), np.int32)
        ctab[np.arange(n)[:, None], idx] = inv.reshape(n, topk).astype(np.int32)
        exp = oracle.mla_attention(bits_host(q), host, ctab, lens, heads, 1, 1.0 / np.sqrt(192.0),
                                   c8=True, indices=idx, sink_k=bits_host(sk), sink_v=bits_host(sv),
                                   threads=THREADS)
    else:
        host = bits_host(cache).reshape(-1, 576)
        exp = oracle.mla_attention(bits_host(q), host, table, lens, heads, bs, 1.0 / np.sqrt(192.0),
                                   window=window, sink_k=bits_host(sk), sink_v=bits_host(sv),
                                   threads=THREADS)
    what = "sparse top-2048" if sparse else "window 2048"
    assert_rel_l2(bf16_host(out), exp, what=what)
    assert_close(bf16_host(out), exp, what=what)


@pytest.mark.parametrize("shape", ["hd256", "page16"])
def test_decode_bench_shapes_full_size(shape):
    """The bench's other GQA decode lines at their size, every sequence against
    the oracle: the Qwen head shape (8 q / 2 kv heads, head_dim 256, block 128)
    and config 2's heads on the reference's 16-token bf16 pages, both over
    config 2's 256 ragged lengths (log-uniform [128, 32768])."""
    import torch
    from ironpangu_amd import ops
    lens = W.decode_meta(0, **W.CONFIGS["decode"]).seq_lens
    if shape == "hd256":
        hq, hd, bs = 8, 256, 128
    else:
        hq, hd, bs = 16, 128, 16
    need = int(((lens.astype(np.int64) + bs - 1) // bs).sum())
    case = W.decode_meta(0, num_seqs=256, lo=128, hi=32768, dist="loguniform", q_heads=hq, kv_heads=2,
                         head_dim=hd, block_size=bs, pool_blocks=need + 64)
    print(f"decode {shape}: {int(case.seq_lens.sum())} tokens", flush=True)
    g = _gen(1100 + hd + bs)
    kc = torch.empty((case.pool_blocks, bs, 2, hd), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    fill_randn(kc, g)
    fill_randn(vc, g)
    q = _randn(g, (256, hq, hd))
    scale = 1.0 / np.sqrt(hd)
    out = ops.paged_decode(q, kc, vc, to_dev(case.block_tables), to_dev(case.seq_lens),
                           case.max_context, scale)
    torch.cuda.synchronize()
    used, ctab = compact_blocks(case.block_tables, case.seq_lens, bs)
    exp = oracle.paged_decode(bits_host(q), _gather_host(kc, used), _gather_host(vc, used), ctab,
                              case.seq_lens, hq, 2, hd, bs, scale, threads=THREADS)
    assert_rel_l2(bf16_host(out), exp, what=f"decode {shape}")
    assert_close(bf16_host(out), exp, what=f"decode {shape}")


def test_config3_mixed_prefill_decode_full_size():
    """Config 3: 8 prefill chunks U[64, 2048] after U[0, 8192] cached tokens plus
    192 decode rows U[256, 16384], one packed varlen call after the slot write of
    every new row. Every decode row is checked, every row of the two longest
    chunks, and of the other chunks the first and last rows and every 31st row;
    a chunk row t sees kv_len - count + t + 1
    keys (native/src/openpangu_attention_metadata.h:20-22), so the oracle checks
    it as a one-row query over that prefix."""
    import torch
    from ironpangu_amd import ops
    case = W.mixed_meta(0)
    nb, bs, hkv, hd, hq = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim, case.q_heads
    tq = int(case.cu_seqlens[-1])
    print(f"config3: {tq} query rows, pool {nb} blocks", flush=True)
    g = _gen(300)
    kc = torch.empty((nb, bs, hkv, hd), dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    fill_randn(kc, g)
    fill_randn(vc, g)
    q = _randn(g, (tq, hq, hd))
    kn = _randn(g, (tq, hkv, hd))
    vn = _randn(g, (tq, hkv, hd))
    k_ref, v_ref = bits_host(kc), bits_host(vc)
    k_before, v_before = kc.clone(), vc.clone()
    slots_d = to_dev(case.slot_mapping.astype(np.int64))
    ops.kv_cache_write(kn, vn, kc, vc, slots_d)
    out = ops.varlen_prefill(q, kc, vc, to_dev(case.block_tables), to_dev(case.cu_seqlens),
                             to_dev(case.kv_lens), case.max_q_len, case.max_kv_len, case.scale)
    torch.cuda.synchronize()
    _check_rows_written_rest_unchanged(kc, k_before, slots_d, kn)
    _check_rows_written_rest_unchanged(vc, v_before, slots_d, vn)
    del k_before, v_before
    oracle.kv_write(bits_host(kn), k_ref, case.slot_mapping)
    oracle.kv_write(bits_host(vn), v_ref, case.slot_mapping)
    rows, seqs, vis = [], [], []
    # every row of the two longest chunks (all eight waves of each of their
    # query tiles), sampled rows of the others
    longest = set(np.argsort(-np.asarray(case.q_lens))[:2].tolist())
    for s in range(len(case.q_lens)):
        start, count, kv = int(case.cu_seqlens[s]), int(case.q_lens[s]), int(case.kv_lens[s])
        ts = set(range(count)) if s in longest else {0, count - 1} | set(range(0, count, 31))
        for t in sorted(ts):
            rows.append(start + t)
            seqs.append(s)
            vis.append(kv - count + t + 1)
    rows = np.array(rows)
    exp = oracle.paged_decode(bits_host(q)[rows], k_ref, v_ref, case.block_tables[np.array(seqs)],
                              np.array(vis, np.int32), hq, hkv, hd, bs, case.scale,
                              threads=THREADS)
    assert_rel_l2(bf16_host(out)[rows], exp, what="config-3 sampled rows")
    assert_close(bf16_host(out)[rows], exp, what="config-3 sampled rows")
    assert len(rows) > 192 + 8 * 3 + sum(sorted(case.q_lens)[-2:])
