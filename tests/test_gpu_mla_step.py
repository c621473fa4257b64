"""GPU: the fused MLA decode step (ifattn_mla_decode_step) against the two
separate launches it replaces: ifattn_mla_norm_rope_cache_write of each
sequence's new row at its last position, then ifattn_mla_decode_{bf16,c8}.
Outputs and the whole cache are required to be bit-identical, on bf16 and
packed C8 rows, over ragged lengths including 1-key and empty sequences and
sequences whose last tile falls in different shares; the written rows are also
checked against the oracle's writer (bit-exact) and the output against the
oracle's decode on the oracle-written cache (1e-2 abs + rel)."""
import numpy as np
import pytest

import oracle
from helpers import assert_close, bf16_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu
f32 = np.float32


def bf(x):
    return W.bf16_bits(np.asarray(x, np.float32))


def case(seed, lens, bs, packed, heads=16):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    n = len(lens)
    need = (lens.astype(np.int64) + bs - 1) // bs
    pool = int(need.sum()) + 4
    stride = int(max(need.max(), 1)) + 1
    table = W.block_tables_for(rng, lens, bs, pool, stride)
    lat = bf(rng.standard_normal((pool * bs, 576)).astype(f32) * f32(0.5))
    cache = oracle.mla_pack_c8(lat).reshape(pool, bs, 656) if packed else lat.reshape(pool, bs, 576)
    q = bf(rng.standard_normal((n, heads, 576)).astype(f32) * f32(0.5))
    x = bf(rng.standard_normal((n, 576)).astype(f32))
    gamma = bf(rng.uniform(0.5, 1.5, 512).astype(f32))
    ang = rng.uniform(0, 6.3, (n, 32)).astype(f32)
    cos = bf(np.concatenate([np.cos(ang), np.cos(ang)], 1))
    sin = bf(np.concatenate([np.sin(ang), np.sin(ang)], 1))
    last = np.maximum(lens - 1, 0)
    slots = np.where(lens > 0, table[np.arange(n), last // bs].astype(np.int64) * bs + last % bs, -1)
    return q, x, gamma, cos, sin, cache, table, lens, slots, stride * bs


@pytest.mark.parametrize("packed", [False, True], ids=["bf16", "c8"])
@pytest.mark.parametrize("seed,lens,bs", [
    (1, [1, 64, 65, 3000, 0, 777, 40000, 5], 64),
    (2, list(np.random.default_rng(9).integers(1, 20000, 96)), 64),
    (3, [33, 4096, 12345, 1, 2], 32),
])
def test_fused_step_equals_writer_then_decode(packed, seed, lens, bs):
    import torch
    from ironpangu_amd import ops
    print(f"mla step packed={packed} seed={seed} n={len(lens)} bs={bs}", flush=True)
    q, x, gamma, cos, sin, cache, table, lens, slots, maxc = case(seed, lens, bs, packed)
    dq, dx, dg, dc, ds = (to_dev(a) for a in (q, x, gamma, cos, sin))
    if packed:
        c1 = to_dev(cache)
    else:
        c1 = to_dev(cache).view(torch.bfloat16)
    c2 = c1.clone()
    dt, dl = to_dev(table), to_dev(lens)
    bfv = lambda t: t.view(torch.bfloat16)
    # separate launches (sequences without keys write nothing in the fused step)
    live = slots >= 0
    if live.any():
        idx = np.nonzero(live)[0]
        ops.mla_norm_rope_cache_write(bfv(to_dev(x[idx])), bfv(dg), bfv(to_dev(cos[idx])),
                                      bfv(to_dev(sin[idx])), c1, to_dev(slots[idx]))
    o1 = ops.mla_decode(bfv(dq), c1, dt, dl, maxc)
    o2 = ops.mla_decode_step(bfv(dq), bfv(dx), bfv(dg), bfv(dc), bfv(ds), c2, dt, dl, maxc)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "outputs differ"
    assert torch.equal(c1.view(torch.uint8), c2.view(torch.uint8)), "caches differ"
    # the written rows against the oracle's writer, and the output against the oracle
    stride = 656 if packed else 1152
    host = cache.reshape(-1).view(np.uint8).reshape(-1, stride).copy()
    if live.any():
        idx = np.nonzero(live)[0]
        host = oracle.mla_norm_rope_write(x[idx], gamma, cos[idx], sin[idx], slots[idx], host, packed)
    got_cache = c2.view(torch.uint8).cpu().numpy().reshape(-1, stride)
    assert np.array_equal(got_cache, host)
    ref_cache = host if packed else host.view(np.uint16).reshape(-1, 576)
    exp = oracle.mla_decode(q, ref_cache, table, lens, 16, bs, 1.0 / np.sqrt(192.0), c8=packed)
    assert_close(bf16_host(o2), exp)


@pytest.mark.parametrize("packed", [False, True], ids=["bf16", "c8"])
def test_fused_step_graph_replay(packed):
    """The fused step captured into a HIP graph: three replays, each with new
    latent rows copied into the captured input and the cache restored, with
    eager calls between them; every replay equals the eager call on the same
    inputs bit for bit (outputs and caches)."""
    import torch
    from ironpangu_amd import ops
    print(f"mla step graph packed={packed}", flush=True)
    lens = list(np.random.default_rng(11).integers(1, 9000, 40)) + [0, 1]
    q, x, gamma, cos, sin, cache, table, lens, slots, maxc = case(21, lens, 64, packed)
    bfv = lambda t: t.view(torch.bfloat16)
    dq, dx, dg, dc, ds = (to_dev(a) for a in (q, x, gamma, cos, sin))
    dt, dl = to_dev(table), to_dev(lens)
    c0 = to_dev(cache) if packed else to_dev(cache).view(torch.bfloat16)
    cg = c0.clone()
    ws = ops.mla_workspace(len(lens), 16, maxc, 64)
    out = torch.empty((len(lens), 16, 512), dtype=torch.bfloat16, device="cuda")

    def step(c, o, xin):
        ops.mla_decode_step(bfv(dq), bfv(xin), bfv(dg), bfv(dc), bfv(ds), c, dt, dl, maxc,
                            out=o, workspace=ws)

    step(cg, out, dx)  # first call on the device before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(cg, out, dx)
    rng = np.random.default_rng(5)
    for r in range(3):
        xr = to_dev(bf(rng.standard_normal((len(lens), 576)).astype(f32)))
        dx.copy_(xr)
        cg.copy_(c0)
        g.replay()
        torch.cuda.synchronize()
        ce = c0.clone()
        oe = torch.empty_like(out)
        ws_e = ops.mla_workspace(len(lens), 16, maxc, 64)
        ops.mla_decode_step(bfv(dq), bfv(xr), bfv(dg), bfv(dc), bfv(ds), ce, dt, dl, maxc,
                            out=oe, workspace=ws_e)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), oe.view(torch.int16)), f"replay {r}: outputs differ"
        assert torch.equal(cg.view(torch.uint8), ce.view(torch.uint8)), f"replay {r}: caches differ"
