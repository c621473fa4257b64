"""GPU: the IFKernelV1 plug-ins (prepare -> enqueue -> release, as the
reference loader drives them) reproduce the direct C-ABI results bit for bit."""
import ctypes as C

import numpy as np
import pytest

from helpers import to_dev
from ironpangu_amd import workloads as W
from test_abi import Prepared, Tensor, load_plugin

pytestmark = pytest.mark.gpu

DT = {"torch.bfloat16": 2, "torch.int8": 1, "torch.float32": 3, "torch.int32": 4,
      "torch.int64": 5, "torch.uint8": 1}


def desc(t, access):
    d = Tensor()
    d.struct_bytes = C.sizeof(Tensor)
    d.dtype = DT[str(t.dtype)]
    d.rank = t.dim()
    d.access = access
    d.data = t.data_ptr()
    d.allocation_bytes = t.numel() * t.element_size()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        d.shape[i] = s
        d.strides[i] = st
    return d


def run(name, ins, outs):
    import torch
    so, entry = load_plugin(name)
    k = entry(2).contents
    a = (Tensor * len(ins))(*[desc(t, acc) for t, acc in ins])
    b = (Tensor * len(outs))(*[desc(t, acc) for t, acc in outs])
    p = Prepared()
    assert k.prepare(a, len(ins), b, len(outs), C.byref(p)) == 0
    ws = torch.empty(max(p.workspace_bytes, 256), dtype=torch.uint8, device="cuda")
    st = k.enqueue(p.state, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    k.release(p.state)
    assert st == 0


def test_plugin_write_and_decode_match_direct():
    import torch
    from ironpangu_amd import ops
    case = W.config_case("cpu_ref", seed=3)
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc1 = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc1 = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    kc2, vc2 = kc1.clone(), vc1.clone()
    kn, vn, q = to_dev(h["k_new"]), to_dev(h["v_new"]), to_dev(h["q"])
    slots = to_dev(case.slot_mapping.astype(np.int64))
    tables, lens = to_dev(case.block_tables), to_dev(case.seq_lens)
    run("kv_cache_write_bf16", [(kn, 1), (vn, 1), (slots, 1)], [(kc1, 3), (vc1, 3)])
    ops.kv_cache_write(kn, vn, kc2, vc2, slots)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    out1 = torch.empty_like(q)
    run("paged_decode_gqa_bf16", [(q, 1), (kc1, 1), (vc1, 1), (tables, 1), (lens, 1)], [(out1, 2)])
    max_ctx = tables.shape[1] * bs
    out2 = ops.paged_decode(q, kc2, vc2, tables, lens, max_ctx, 1.0 / np.sqrt(hd))
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_plugin_mla_c8_write_and_decode():
    import torch
    from ironpangu_amd import ops
    case = W.mla_host_case(4, num_seqs=3, lo=10, hi=700, dist="uniform", heads=16, block_size=64)
    h = case.host
    cache1 = torch.zeros((case.pool_blocks, 64, 656), dtype=torch.int8, device="cuda")
    allslots = torch.arange(case.pool_blocks * 64, dtype=torch.int64, device="cuda")
    run("mla_cache_write_c8", [(to_dev(h["pool"]), 1), (allslots, 1)], [(cache1, 3)])
    cache2 = torch.zeros((case.pool_blocks, 64, 656), dtype=torch.uint8, device="cuda")
    ops.mla_cache_write_c8(to_dev(h["pool"]), cache2, allslots)
    torch.cuda.synchronize()
    assert torch.equal(cache1.view(torch.uint8), cache2)
    q, tables, lens = to_dev(h["q"]), to_dev(case.block_tables), to_dev(case.seq_lens)
    out1 = torch.empty((3, 16, 512), dtype=torch.bfloat16, device="cuda")
    run("mla_decode_c8", [(q, 1), (cache1, 1), (tables, 1), (lens, 1)], [(out1, 2)])
    out2 = ops.mla_decode(q, cache2, tables, lens, tables.shape[1] * 64, 1.0 / np.sqrt(192.0))
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_plugin_norm_rope_write_and_attention_contracts():
    """Fused writer (C8), sparse C8 attention with sinks and the w512 window
    contract, each against the direct call."""
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(21)
    rows, nslots = 64, 2048
    x = to_dev(W.bf16_randn(rng, (rows, 576)))
    g = to_dev(W.bf16_randn(rng, (512,)))
    cs, sn = to_dev(W.bf16_randn(rng, (rows, 64))), to_dev(W.bf16_randn(rng, (rows, 64)))
    slots = torch.from_numpy(rng.permutation(nslots)[:rows].astype(np.int64)).cuda()
    c1 = torch.zeros((nslots // 32, 32, 656), dtype=torch.int8, device="cuda")
    c2 = torch.zeros((nslots // 32, 32, 656), dtype=torch.uint8, device="cuda")
    run("mla_norm_rope_cache_c8", [(x, 1), (g, 1), (cs, 1), (sn, 1), (slots, 1)], [(c1, 3)])
    ops.mla_norm_rope_cache_write(x, g, cs, sn, c2, slots)
    torch.cuda.synchronize()
    assert torch.equal(c1.view(torch.uint8), c2)

    # sparse C8 attention over the written cache: 2 sequences, 3 + 2 rows
    pool = W.bf16_randn(rng, (nslots, 576), std=0.5)
    ops.mla_cache_write_c8(to_dev(pool), c2, torch.arange(nslots, dtype=torch.int64, device="cuda"))
    table = torch.from_numpy(rng.permutation(64).astype(np.int32).reshape(2, 32)).cuda()
    cu = torch.tensor([0, 3, 5], dtype=torch.int32, device="cuda")
    kv = torch.tensor([900, 400], dtype=torch.int32, device="cuda")
    topk = 512
    idx = np.full((5, topk), -1, np.int32)
    for t, causal in enumerate([898, 899, 900, 399, 400]):
        n = min(causal, topk)
        idx[t, :n] = rng.choice(causal, n, replace=False)
    idx = torch.from_numpy(idx).cuda()
    q = to_dev(W.bf16_randn(rng, (5, 6, 576), std=0.5))
    sk, sv = to_dev(W.bf16_randn(rng, (128, 576))), to_dev(W.bf16_randn(rng, (128, 512)))
    o1 = torch.empty((5, 6, 512), dtype=torch.bfloat16, device="cuda")
    run("mla_sparse_attention_c8", [(q, 1), (c2.view(torch.int8), 1), (idx, 1), (table, 1), (cu, 1),
                                    (kv, 1), (sk, 1), (sv, 1)], [(o1, 2)])
    o2 = ops.mla_attention(q, c2, table, kv, 1024, cu_seqlens=cu, indices=idx, sink_keys=sk,
                           sink_values=sv)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)

    # w512 window over a bf16 cache with 16-token pages
    cb = to_dev(pool).view(nslots // 16, 16, 576)
    table16 = torch.from_numpy(rng.permutation(128).astype(np.int32).reshape(2, 64)).cuda()
    o3 = torch.empty_like(o1)
    run("mla_window_attention_w512_bf16", [(q, 1), (cb, 1), (table16, 1), (cu, 1), (kv, 1), (sk, 1),
                                           (sv, 1)], [(o3, 2)])
    o4 = ops.mla_attention(q, cb, table16, kv, 1024, cu_seqlens=cu, window=512, sink_keys=sk,
                           sink_values=sv)
    torch.cuda.synchronize()
    assert torch.equal(o3, o4)
