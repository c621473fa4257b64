"""GPU: the allocation-free decode step (ifattn_paged_decode_step_bf16_noalloc,
a static device scratch in place of the workspace) against the workspace entry
point ifattn_paged_decode_step_bf16, bit for bit: outputs and caches, on two
calls in a row with the second smaller, plus the size rejection."""
import ctypes as C

import numpy as np
import pytest

from helpers import to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _step(noalloc, case, h, kc, vc, out):
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd._native import check, lib
    q, kn, vn = to_dev(h["q"]), to_dev(h["k_new"]), to_dev(h["v_new"])
    slots = to_dev(case.slot_mapping.astype(np.int64))
    tables, lens = to_dev(case.block_tables), to_dev(case.seq_lens)
    nb, bs, hkv, hd = kc.shape
    args = [q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(),
            slots.data_ptr(), 5, case.num_seqs, tables.data_ptr(), tables.shape[1], lens.data_ptr(),
            out.data_ptr(), case.num_seqs, case.q_heads, hkv, hd, bs, nb, case.max_context,
            case.scale]
    s = torch.cuda.current_stream().cuda_stream
    if noalloc:
        check(lib().ifattn_paged_decode_step_bf16_noalloc(*args, s), "noalloc step")
    else:
        ws = ops.decode_workspace(case.num_seqs, case.q_heads, hd, case.max_context)
        check(lib().ifattn_paged_decode_step_bf16(*args, ws.data_ptr(), ws.numel(), s), "step")
    torch.cuda.synchronize()


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_step_matches_workspace_step(order):
    import torch
    # call 1: 64 sequences up to 20000 tokens (split-K partials in the scratch);
    # call 2: 5 shorter sequences, so stale scratch contents must not leak in
    for seed, n, hi in ((3, 64, 20000), (4, 5, 3000)):
        print(f"noalloc case seed={seed} seqs={n} hi={hi}", flush=True)
        case = W.decode_host_case(seed, num_seqs=n, lo=1, hi=hi, dist="loguniform", q_heads=16,
                                  kv_heads=2, head_dim=128, block_size=128,
                                  pool_blocks=n * ((hi + 127) // 128) + 4)
        h = case.host
        shape = (case.pool_blocks, 128, 2, 128)
        k1, v1 = to_dev(h["k_pool"]).view(shape), to_dev(h["v_pool"]).view(shape)
        k2, v2 = k1.clone(), v1.clone()
        o1 = torch.empty((n, 16, 128), dtype=torch.bfloat16, device="cuda")
        o2 = torch.empty_like(o1)
        _step(False, case, h, k1, v1, o1)
        _step(True, case, h, k2, v2, o2)
        assert torch.equal(o1, o2), "outputs differ"
        assert torch.equal(k1, k2) and torch.equal(v1, v2), "caches differ"


def test_noalloc_step_rejects_calls_beyond_the_scratch():
    from ironpangu_amd._native import lib
    l = lib()
    # partials for 128 q heads of 256 dims (two shares per persistent workgroup)
    # take far more than 32 MiB
    need = l.ifattn_paged_decode_workspace_size(64, 128, 256, 4096)
    assert need > (32 << 20)
    a = 0x10000
    st = l.ifattn_paged_decode_step_bf16_noalloc(a, a, a, a, a, a, 5, 64, a, 32, a, a, 64,
                                                 128, 8, 256, 128, 1 << 20, 4096, 0.1, None)
    assert st == -1 and b"32 MiB" in l.ifattn_last_error()


def test_noalloc_step_under_graph_capture():
    """The entry point recorded into a HIP graph (after one eager warm-up call,
    which also looks up the scratch address) and replayed three times, with
    eager work and synchronisation between replays: every replay equals the
    workspace entry point's eager result bit for bit."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd._native import check, lib
    case = W.decode_host_case(9, num_seqs=32, lo=1, hi=9000, dist="loguniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=128,
                              pool_blocks=32 * ((9000 + 127) // 128) + 4)
    h = case.host
    shape = (case.pool_blocks, 128, 2, 128)
    k_ref, v_ref = to_dev(h["k_pool"]).view(shape), to_dev(h["v_pool"]).view(shape)
    k_g, v_g = k_ref.clone(), v_ref.clone()
    o_ref = torch.empty((32, 16, 128), dtype=torch.bfloat16, device="cuda")
    _step(False, case, h, k_ref, v_ref, o_ref)
    q, kn, vn = to_dev(h["q"]), to_dev(h["k_new"]), to_dev(h["v_new"])
    slots = to_dev(case.slot_mapping.astype(np.int64))
    tables, lens = to_dev(case.block_tables), to_dev(case.seq_lens)
    out = torch.empty_like(o_ref)
    args = [q.data_ptr(), kn.data_ptr(), vn.data_ptr(), k_g.data_ptr(), v_g.data_ptr(),
            slots.data_ptr(), 5, 32, tables.data_ptr(), tables.shape[1], lens.data_ptr(),
            out.data_ptr(), 32, 16, 2, 128, 128, case.pool_blocks, case.max_context, case.scale]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        check(lib().ifattn_paged_decode_step_bf16_noalloc(*args, s.cuda_stream), "warm-up")
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            check(lib().ifattn_paged_decode_step_bf16_noalloc(*args, s.cuda_stream), "capture")
    for rep in range(3):
        out.fill_(0)                      # eager work between replays
        scratch_user = torch.empty_like(o_ref)
        _step(True, case, h, k_g.clone(), v_g.clone(), scratch_user)  # eager call reuses the scratch
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, o_ref), f"replay {rep}: outputs differ"
        assert torch.equal(k_g, k_ref) and torch.equal(v_g, v_ref), f"replay {rep}: caches differ"
