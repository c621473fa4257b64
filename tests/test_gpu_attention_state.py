"""GPU: the attention-state object drives the MLA attention over its own
buffers (include/ifattn_state.h; AttentionState, native/src/openpangu_decoder_state.h:16-48).
Rows are written through the state's append() slots, the table is uploaded
from blocks(), and attend() equals the direct C-ABI call on the same buffers bit
for bit and the oracle within 1e-2 abs + rel."""
import numpy as np
import pytest

import oracle
from helpers import assert_close, bf16_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu


class _Dev:
    """torch view of a raw device buffer (CUDA array interface)."""

    def __init__(self, ptr, shape, typestr):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr,
                                         "data": (int(ptr), False), "version": 3, "strides": None}


def view(ptr, shape, dtype):
    import torch
    typestr = {torch.int16: "<i2", torch.int32: "<i4", torch.uint8: "|u1", torch.float32: "<f4"}[dtype]
    return torch.as_tensor(_Dev(ptr, shape, typestr), device="cuda")


@pytest.mark.parametrize("packed", [False, True], ids=["bf16_window", "c8_sparse"])
def test_state_attend_matches_direct_and_oracle(packed):
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd.host import AttentionState
    heads, cap, residents = 6, 4096, 2
    context = 0 if packed else 8192   # bf16: ring table over a 4096-token page set
    s = AttentionState(16, cap, packed, residents, True, context, heads)
    g = s.geometry
    page, entries, nb = g["page_tokens"], g["table_entries"], g["num_blocks"]
    b = s.buffers()
    rng = np.random.default_rng(11 + int(packed))
    # resident 1 serves the query; its pages are a random permutation of its own
    s.page_binding.select(1)
    per = cap // page
    s.page_binding.bind((rng.permutation(per) + per).astype(np.int32))
    kv_len = 5000 if not packed else 3000
    positions = np.arange(kv_len - (cap if context else kv_len), kv_len) if context else np.arange(kv_len)
    positions = positions[positions >= 0]
    slots = np.array([s.append(int(p)) for p in positions], np.int64)
    rows = W.bf16_randn(rng, (len(slots), 576), std=0.5)
    if packed:
        cache = view(b["cache"], (nb, page, 656), torch.uint8)
        ops.mla_cache_write_c8(to_dev(rows), cache, to_dev(slots))
    else:
        cache = view(b["cache"], (nb, page, 576), torch.int16).view(torch.bfloat16)
        ops.kv_cache_write(to_dev(rows), None, cache, None, to_dev(slots))
    q = W.bf16_randn(rng, (1, heads, 576), std=0.5)
    view(b["query"], (1, heads, 576), torch.int16).copy_(to_dev(q).view(torch.int16))
    sk, sv = W.bf16_randn(rng, (128, 576), std=0.5), W.bf16_randn(rng, (128, 512), std=0.5)
    view(b["sink_keys"], (128, 576), torch.int16).copy_(to_dev(sk).view(torch.int16))
    view(b["sink_values"], (128, 512), torch.int16).copy_(to_dev(sv).view(torch.int16))
    idx = None
    if packed:
        idx = np.full((1, 512), -1, np.int32)
        idx[0, :500] = rng.choice(kv_len, 500, replace=False)
        view(b["indices"], (1, 512), torch.int32).copy_(to_dev(idx))
    stream = torch.cuda.current_stream().cuda_stream
    s.upload_table(stream)
    s.set_length(kv_len, stream)
    window = 0 if packed else 2048
    s.attend(window=window, sinks=True, stream=stream)
    torch.cuda.synchronize()
    out = view(b["out"], (1, heads, 512), torch.int16).view(torch.bfloat16).clone()
    # direct call over the same buffers
    table = view(b["table"], (1, entries), torch.int32)
    kv = view(b["kv_len"], (1,), torch.int32)
    direct = ops.mla_attention(to_dev(q), cache, table, kv, entries * page,
                               indices=to_dev(idx) if packed else None, window=window,
                               sink_keys=to_dev(sk), sink_values=to_dev(sv))
    torch.cuda.synchronize()
    assert torch.equal(out, direct)
    # the uploaded table is blocks()
    assert np.array_equal(table.cpu().numpy()[0], s.blocks())
    host_cache = cache.view(torch.uint8).cpu().numpy() if packed else \
        cache.view(torch.int16).cpu().numpy().view(np.uint16)
    exp = oracle.mla_attention(q, host_cache, s.blocks()[None, :], np.array([kv_len], np.int32), heads,
                               page, 1.0 / np.sqrt(192.0), c8=packed, indices=idx, window=window,
                               sink_k=sk, sink_v=sv)
    assert_close(bf16_host(out), exp)
