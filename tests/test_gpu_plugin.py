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
