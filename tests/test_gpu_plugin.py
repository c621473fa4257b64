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


def _ref_run(name, contract, ins, outs):
    """prepare -> enqueue -> release through the reference's own loader
    (native/src/compiled_kernel.cpp, compiled in place), version 1 descriptors:
    integer tensors as I8 byte views, in-place caches as write outputs."""
    import torch
    from test_abi import ref_open, ref_prepare
    st, h, l = ref_open(name, contract)
    assert st == 0, l.ref_loader_error()

    def v1(t, access):
        if t.dtype in (torch.int32, torch.int64):
            t = t.view(torch.int8)  # byte view: last extent x4 / x8
        return desc(t, access)

    st, p, ws = ref_prepare(l, h, [v1(t, a) for t, a in ins], [v1(t, a) for t, a in outs])
    assert st == 0, l.ref_loader_error()
    w = torch.empty(max(ws, 256), dtype=torch.uint8, device="cuda")
    st = l.ref_loader_enqueue(p, w.data_ptr(), w.numel(), torch.cuda.current_stream().cuda_stream)
    assert st == 0, l.ref_loader_error()
    torch.cuda.synchronize()
    l.ref_loader_release(p)
    l.ref_loader_close(h)


def test_reference_loader_v1_write_decode_prefill_match_direct():
    import torch
    from ironpangu_amd import ops
    case = W.config_case("cpu_ref", seed=8)
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc1 = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc1 = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    kc2, vc2 = kc1.clone(), vc1.clone()
    kn, vn, q = to_dev(h["k_new"]), to_dev(h["v_new"]), to_dev(h["q"])
    slots = to_dev(case.slot_mapping.astype(np.int64))
    tables, lens = to_dev(case.block_tables), to_dev(case.seq_lens)
    _ref_run("kv_cache_write_bf16", "inferfabric.kv_cache_write.bf16.v1",
             [(kn, 1), (vn, 1), (slots, 1)], [(kc1, 2), (vc1, 2)])
    ops.kv_cache_write(kn, vn, kc2, vc2, slots)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    out1 = torch.empty_like(q)
    _ref_run("paged_decode_gqa_bf16", "inferfabric.paged_decode.gqa.bf16.v1",
             [(q, 1), (kc1, 1), (vc1, 1), (tables, 1), (lens, 1)], [(out1, 2)])
    out2 = ops.paged_decode(q, kc2, vc2, tables, lens, tables.shape[1] * bs, 1.0 / np.sqrt(hd))
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    # packed varlen prefill: one 5-row chunk and one decode row over the same caches
    cu = torch.tensor([0, 5, 6], dtype=torch.int32, device="cuda")
    kv = torch.tensor([int(case.seq_lens[0]), int(case.seq_lens[1])], dtype=torch.int32, device="cuda")
    qp = q[:6].contiguous()
    o1 = torch.empty_like(qp)
    _ref_run("varlen_prefill_bf16", "inferfabric.varlen_prefill.bf16.v1",
             [(qp, 1), (kc1, 1), (vc1, 1), (tables[:2].contiguous(), 1), (cu, 1), (kv, 1)], [(o1, 2)])
    o2 = ops.varlen_prefill(qp, kc2, vc2, tables[:2].contiguous(), cu, kv, 6, tables.shape[1] * bs)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_plugin_gated_attention_matches_direct():
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(31)
    batch, context, nslots = 5, 1500, 8192
    q = to_dev(W.bf16_randn(rng, (batch, 8, 256)))
    k, v = to_dev(W.bf16_randn(rng, (batch, 512))), to_dev(W.bf16_randn(rng, (batch, 512)))
    gate = to_dev(W.bf16_randn(rng, (batch, 8, 256)))
    keys1 = to_dev(W.bf16_randn(rng, (nslots, 512)))
    vals1 = to_dev(W.bf16_randn(rng, (nslots, 512)))
    keys2, vals2 = keys1.clone(), vals1.clone()
    append = torch.from_numpy(rng.permutation(nslots)[:batch].astype(np.int64)).cuda()
    table = torch.from_numpy(rng.integers(0, nslots, (batch, context)).astype(np.int64)).cuda()
    mask = torch.from_numpy(np.where(rng.random((batch, context)) < 0.2, -np.inf, 0.0)
                            .astype(np.float32)).cuda()
    o1 = torch.empty_like(q)
    run("paged_attention_qwen_gated_bf16",
        [(q, 1), (k, 1), (v, 1), (gate, 1), (append, 1), (table, 1), (mask, 1)],
        [(keys1, 3), (vals1, 3), (o1, 2)])
    o2 = ops.gated_paged_attention(q, k, v, gate, keys2, vals2, append, table, mask)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(keys1, keys2) and torch.equal(vals1, vals2)
