"""HIP-graph capture of the MLA attention, varlen prefill and fused writer
paths: each captured call is replayed several times with new device-side
metadata (lengths, index lists) written between replays, eager work and
synchronisation in between; every replay must equal an eager call on the same
metadata bit for bit (the plans are read on the device, no host reads)."""
import numpy as np
import pytest

import oracle
from helpers import to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _replays(capture, update, eager, n=3):
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        capture()  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = capture()
    for i in range(n):
        update(i)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = eager()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from eager"


def test_graph_mla_window_and_sparse():
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(31)
    bs, nb, heads = 32, 96, 6
    lens = np.array([700, 1500, 40], np.int32)
    table = torch.from_numpy(rng.permutation(nb).astype(np.int32).reshape(3, 32)).cuda()
    cache = to_dev(W.bf16_randn(rng, (nb * bs, 576), std=0.5)).view(nb, bs, 576)
    c8 = torch.zeros((nb, bs, 656), dtype=torch.uint8, device="cuda")
    ops.mla_cache_write_c8(cache.view(-1, 576), c8, torch.arange(nb * bs, dtype=torch.int64, device="cuda"))
    q = to_dev(W.bf16_randn(rng, (5, heads, 576), std=0.5))
    cu = torch.tensor([0, 2, 4, 5], dtype=torch.int32, device="cuda")
    kv = torch.from_numpy(lens).cuda()
    sk, sv = to_dev(W.bf16_randn(rng, (128, 576))), to_dev(W.bf16_randn(rng, (128, 512)))
    idx = torch.full((5, 512), -1, dtype=torch.int32, device="cuda")

    def set_meta(i):
        new = lens - 7 * i
        kv.copy_(torch.from_numpy(new))
        rows = []
        for s, (a, b) in enumerate([(0, 2), (2, 4), (4, 5)]):
            for t in range(a, b):
                causal = int(new[s]) - (b - a) + (t - a) + 1
                r = np.full(512, -1, np.int32)
                n = min(causal, 512)
                r[:n] = rng.choice(causal, n, replace=False)
                rows.append(r)
        idx.copy_(torch.from_numpy(np.stack(rows)))

    set_meta(0)
    ws_w = torch.empty(int(ops.lib().ifattn_mla_attention_workspace_size(5, heads, 1024, 300, 0, 128, bs)),
                       dtype=torch.uint8, device="cuda")
    ws_s = torch.empty(int(ops.lib().ifattn_mla_attention_workspace_size(5, heads, 1024, 0, 512, 128, bs)),
                       dtype=torch.uint8, device="cuda")
    out_w = torch.empty((5, heads, 512), dtype=torch.bfloat16, device="cuda")
    out_s = torch.empty_like(out_w)

    def window():
        return ops.mla_attention(q, cache, table, kv, 1024, cu_seqlens=cu, window=300, sink_keys=sk,
                                 sink_values=sv, out=out_w, workspace=ws_w)

    def sparse():
        return ops.mla_attention(q, c8, table, kv, 1024, cu_seqlens=cu, indices=idx, sink_keys=sk,
                                 sink_values=sv, out=out_s, workspace=ws_s)

    _replays(window, set_meta, lambda: ops.mla_attention(q, cache, table, kv, 1024, cu_seqlens=cu,
                                                          window=300, sink_keys=sk, sink_values=sv))
    _replays(sparse, set_meta, lambda: ops.mla_attention(q, c8, table, kv, 1024, cu_seqlens=cu,
                                                          indices=idx, sink_keys=sk, sink_values=sv))


def test_graph_mla_wide_layout():
    """A dense bf16 call with at least 2^18 possible keys (rows x max_context)
    runs the two-workgroup layout, whose workgroups write the plan into the
    workspace themselves: replays with new lengths equal eager calls."""
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(37)
    bs, nb, heads, maxc = 32, 96, 6, 65536
    lens = np.array([700, 1500, 40], np.int32)
    assert 5 * maxc >= 1 << 18
    table = torch.from_numpy(rng.integers(0, nb, (3, maxc // bs)).astype(np.int32)).cuda()
    cache = to_dev(W.bf16_randn(rng, (nb * bs, 576), std=0.5)).view(nb, bs, 576)
    q = to_dev(W.bf16_randn(rng, (5, heads, 576), std=0.5))
    cu = torch.tensor([0, 2, 4, 5], dtype=torch.int32, device="cuda")
    kv = torch.from_numpy(lens).cuda()
    sk, sv = to_dev(W.bf16_randn(rng, (128, 576))), to_dev(W.bf16_randn(rng, (128, 512)))

    def set_meta(i):
        kv.copy_(torch.from_numpy(lens + 301 * i))

    ws = torch.empty(int(ops.lib().ifattn_mla_attention_workspace_size(5, heads, maxc, 0, 0, 128, bs)),
                     dtype=torch.uint8, device="cuda")
    out = torch.empty((5, heads, 512), dtype=torch.bfloat16, device="cuda")

    def call():
        return ops.mla_attention(q, cache, table, kv, maxc, cu_seqlens=cu, sink_keys=sk, sink_values=sv,
                                 out=out, workspace=ws)

    _replays(call, set_meta, lambda: ops.mla_attention(q, cache, table, kv, maxc, cu_seqlens=cu,
                                                        sink_keys=sk, sink_values=sv))


def test_graph_varlen_prefill():
    import torch
    from ironpangu_amd import ops
    case = W.mixed_host_case(5, n_chunks=3, chunk_lo=40, chunk_hi=300, prior_lo=0, prior_hi=900,
                             n_decode=4, dec_lo=50, dec_hi=2000)
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    q = to_dev(h["q"])
    tables = to_dev(case.block_tables)
    cu = to_dev(case.cu_seqlens)
    kv = to_dev(case.kv_lens)
    base = case.kv_lens.copy()
    ws = ops.prefill_workspace(len(case.q_lens), int(case.cu_seqlens[-1]), case.q_heads, hd,
                               case.max_kv_len)
    out = torch.empty_like(q)

    def call(o=None, w=None):
        return ops.varlen_prefill(q, kc, vc, tables, cu, kv, case.max_q_len, case.max_kv_len,
                                  case.scale, out=o, workspace=w)

    def update(i):  # shorter cached prefixes on later replays
        kv.copy_(torch.from_numpy(np.maximum(base - 13 * i, case.q_lens)).cuda())

    _replays(lambda: call(out, ws), update, lambda: call())


def test_graph_norm_rope_write():
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(8)
    rows = 40
    x = to_dev(W.bf16_randn(rng, (rows, 576)))
    g = to_dev(W.bf16_randn(rng, (512,)))
    cs, sn = to_dev(W.bf16_randn(rng, (rows, 64))), to_dev(W.bf16_randn(rng, (rows, 64)))
    slots = torch.zeros(rows, dtype=torch.int64, device="cuda")
    cache = torch.zeros((64, 32, 656), dtype=torch.uint8, device="cuda")

    def write():
        ops.mla_norm_rope_cache_write(x, g, cs, sn, cache, slots)
        return cache

    def update(i):
        slots.copy_(torch.from_numpy(rng.permutation(2048)[:rows].astype(np.int64)).cuda())
        cache.zero_()

    def eager():
        ref = torch.zeros_like(cache)
        ops.mla_norm_rope_cache_write(x, g, cs, sn, ref, slots)
        return ref

    _replays(write, update, eager)


@pytest.mark.parametrize("bits", [8, 4])
def test_graph_legacy_quantize_position_replay(bits):
    """if_cache_quantize captured once: each replay reads the device position
    written before it and fills that row (cache_quantization_probe.cpp:23-34
    replays with a changed position); rows written by earlier replays stay."""
    import torch
    from ironpangu_amd import ops
    width, rows = 576, 64
    rng = np.random.default_rng(41)
    xs = [W.bf16_randn(rng, (width,)) for _ in range(3)]
    x = torch.empty(width, dtype=torch.bfloat16, device="cuda")
    packed = torch.zeros((rows * width * bits // 8,), dtype=torch.uint8, device="cuda")
    scales = torch.ones(rows, dtype=torch.float32, device="cuda")
    pos = torch.zeros(1, dtype=torch.int64, device="cuda")
    x.copy_(to_dev(xs[0]))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.cache_quantize(x, packed, scales, pos, bits)  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.cache_quantize(x, packed, scales, pos, bits)
    placed = {}
    for i, row in enumerate((5, 17, 63)):
        x.copy_(to_dev(xs[i]))
        pos.fill_(row)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        placed[row] = oracle.quant_legacy(xs[i], bits)
        p = packed.cpu().numpy().reshape(rows, -1)
        sc = scales.cpu().numpy()
        for r, (ref_packed, ref_scale) in placed.items():
            assert np.array_equal(p[r], ref_packed), f"replay {i}: row {r}"
            assert sc[r] == np.float32(ref_scale)
