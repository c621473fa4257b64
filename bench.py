"""Benchmark: one step of the continuous-batching decode path on one MI355X.

A step is the slot-mapped write of the 256 new K/V rows followed by ragged
paged GQA decode attention over 256 sequences (context
log-uniform in [128, 32768], 16 q / 2 kv heads, head_dim 128, block 128,
random block tables over a 65536-block bf16 pool). Inputs are resident in HBM
before the timed region. Prints one JSON line (rank 0).

value  = algorithmic bytes of the step / step time  (GB/s)
roofline: the attention operator's algorithmic bytes / its average duration
          measured with HIP events on the launch stream, against 8 TB/s.
cpu_baseline: the C++ CPU oracle (a restatement of the reference's CPU
          algorithm) timed on this host over a bounded sample of the workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
TRAFFIC_PROFILE = ROOT / "profiles" / "hbm_traffic_decode_kernels.md"


def measured_traffic():
    """HBM bytes per launch of the config-2 decode kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (scaled by the copy calibration)."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch paged_decode_kernel config2:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-seqs", type=int, default=64)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (counter calibration)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip configs 3-5 (reported under 'secondary')")
    ap.add_argument("--only", choices=sorted(SECONDARY),
                    help="run one secondary workload alone and print its JSON (profiling)")
    return ap.parse_args()


def gpu_workload(seed):
    import torch
    from ironpangu_amd import workloads as W
    kw = dict(W.CONFIGS["decode"])
    case = W.decode_meta(seed, **kw)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    nslot = case.pool_blocks * case.block_size
    shape = (case.pool_blocks, case.block_size, case.kv_heads, case.head_dim)

    def randn(*s):
        return torch.randn(*s, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)

    k_cache = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    v_cache = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    # fill in slabs to bound the fp32 temporary
    for t in (k_cache, v_cache):
        flat = t.view(-1)
        step = 1 << 28
        for i in range(0, flat.numel(), step):
            n = min(step, flat.numel() - i)
            flat[i:i + n] = randn(n)
    q = randn(case.num_seqs, case.q_heads, case.head_dim)
    k_new = randn(case.num_seqs, case.kv_heads, case.head_dim)
    v_new = randn(case.num_seqs, case.kv_heads, case.head_dim)
    t = {
        "q": q, "k_new": k_new, "v_new": v_new, "k_cache": k_cache, "v_cache": v_cache,
        "tables": torch.from_numpy(case.block_tables).to(dev),
        "lens": torch.from_numpy(case.seq_lens).to(dev),
        "slots": torch.from_numpy(case.slot_mapping.astype(np.int64)).to(dev),
    }
    del nslot
    return case, t


def cpu_baseline(seed, sample_seqs):
    """Time the CPU oracle on the first `sample_seqs` sequences of the same
    length distribution (bounded sample), with this host's CPU share."""
    import oracle
    from ironpangu_amd import workloads as W
    kw = dict(W.CONFIGS["decode"])
    full = W.decode_meta(seed, **kw)
    lens = full.seq_lens[:sample_seqs].copy()
    bs, hkv, hd, hq = full.block_size, full.kv_heads, full.head_dim, full.q_heads
    rng = np.random.default_rng(seed + 7)
    need = int(((lens + bs - 1) // bs).sum())
    table = W.block_tables_for(rng, lens, bs, need, full.block_tables.shape[1])
    nslot = need * bs
    k = W.bf16_randn(rng, (nslot, hkv, hd))
    v = W.bf16_randn(rng, (nslot, hkv, hd))
    q = W.bf16_randn(rng, (len(lens), hq, hd))
    host_cores = os.cpu_count() or 1
    threads = max(1, min(16, host_cores))  # the box's CPU share for one GPU
    oracle.paged_decode(q, k, v, table, np.minimum(lens, 64), hq, hkv, hd, bs, full.scale,
                        threads=threads)  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        oracle.paged_decode(q, k, v, table, lens, hq, hkv, hd, bs, full.scale, threads=threads)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 400:  # about 10 s of CPU work
            break
    dt = (time.perf_counter() - t0) / reps
    b = W.decode_bytes(lens, hq, hkv, hd, bs, with_write=False)["attention"]
    return {"value": round(b / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "host_cores": host_cores,
            "cores_note": "threads used (capped at the 16-core CPU share of one GPU); "
                          "host_cores is what the host reports", "kind": "port",
            "tokens_per_s": round(len(lens) / dt, 1), "seconds_per_pass": round(dt, 4),
            "sample": f"oracle_paged_decode (fp32 C++ restatement) over the first {len(lens)} of "
                      f"the 256 config-2 sequences ({int(lens.sum())} context tokens), "
                      f"{reps} passes"}


def timed(fn, steps, warmup, graph=False):
    """Average ms of fn() over `steps` back-to-back runs (optionally replayed
    from a HIP graph)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    run = fn
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        run = g.replay
        for _ in range(2):
            run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        run()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def fill_randn(t, gen, std=1.0, clip=None):
    import torch
    flat = t.view(-1)
    step = 1 << 27
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        x = torch.randn(n, generator=gen, device=t.device, dtype=torch.float32) * std
        if clip is not None:
            x.clamp_(-clip, clip)
        flat[i:i + n] = x.to(t.dtype)


def bench_c8(seed, steps, warmup):
    """Config 4: C8 paged decode, 256 seqs, L ~ U[1024,16384]; the pool is
    quantized by the C8 write from N(0,1) clipped to +-4."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    kw = dict(W.CONFIGS["c8"])
    case = W.decode_meta(seed, c8=True, **kw)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 4)
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc = torch.empty((nb, bs, hkv, hd), dtype=torch.int8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty((nb, bs, hkv), dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    rows = 1 << 18
    src_k = torch.empty((rows, hkv, hd), dtype=torch.bfloat16, device=dev)
    src_v = torch.empty_like(src_k)
    for r0 in range(0, nb * bs, rows):
        fill_randn(src_k, g, clip=4.0)
        fill_randn(src_v, g, clip=4.0)
        sl = torch.arange(r0, r0 + rows, dtype=torch.int64, device=dev)
        ops.kv_cache_write_c8(src_k, src_v, kc, vc, ks, vs, sl)
    del src_k, src_v
    q = torch.randn((case.num_seqs, case.q_heads, hd), generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn((case.num_seqs, hkv, hd), generator=g, device=dev).clamp_(-4, 4).to(torch.bfloat16)
    vn = torch.randn((case.num_seqs, hkv, hd), generator=g, device=dev).clamp_(-4, 4).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens = torch.from_numpy(case.seq_lens).to(dev)
    slots = torch.from_numpy(case.slot_mapping.astype(np.int64)).to(dev)
    ws = ops.decode_workspace(case.num_seqs, case.q_heads, hd, case.max_context)
    out = torch.empty_like(q)

    def attn():
        ops.paged_decode(q, kc, vc, tables, lens, case.max_context, case.scale, out=out,
                         workspace=ws, k_scale=ks, v_scale=vs)

    def step():
        ops.kv_cache_write_c8(kn, vn, kc, vc, ks, vs, slots)
        attn()

    ms_step = timed(step, steps, warmup)
    ms_attn = timed(attn, steps, warmup)
    b = W.decode_bytes(case.seq_lens, case.q_heads, hkv, hd, bs, elem_bytes=1, scale_bytes=4)
    res = {"workload": "C8 paged decode, 256 seqs, L~U[1024,16384] (BASELINE config 4)",
           "value": round(b["total"] / ms_step / 1e6, 2), "unit": "GB/s",
           "ms_per_step": round(ms_step, 5), "tokens_per_s": round(case.num_seqs / ms_step * 1e3, 1),
           "total_context_tokens": int(case.seq_lens.sum()),
           "roofline": {"bound": "hbm", "kernel": "paged_decode c8 operator",
                        "achieved": round(b["attention"] / ms_attn / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(b["attention"] / ms_attn / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms_attn, 5), "algorithmic_bytes": b["attention"]}}
    del kc, vc, ks, vs
    torch.cuda.empty_cache()
    return res


def bench_decode_hd256(seed, steps, warmup):
    """GQA decode at the reference Qwen path's head shape (8 q / 2 kv heads,
    head_dim 256; native/src/inferfabric_acl.cpp:1343-1430) over config 2's
    ragged lengths: 256 seqs, log-uniform [128, 32768], block 128."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    rng_lens = W.decode_meta(seed, **W.CONFIGS["decode"]).seq_lens
    need = int(((rng_lens.astype(np.int64) + 127) // 128).sum())
    case = W.decode_meta(seed, num_seqs=256, lo=128, hi=32768, dist="loguniform", q_heads=8,
                         kv_heads=2, head_dim=256, block_size=128, pool_blocks=need + 64)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 7)
    shape = (case.pool_blocks, 128, 2, 256)
    kc = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    fill_randn(kc, g)
    fill_randn(vc, g)
    q = torch.randn((256, 8, 256), generator=g, device=dev).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens = torch.from_numpy(case.seq_lens).to(dev)
    ws = ops.decode_workspace(256, 8, 256, case.max_context)
    out = torch.empty_like(q)

    def attn():
        ops.paged_decode(q, kc, vc, tables, lens, case.max_context, 1.0 / 16.0, out=out, workspace=ws)

    ms = timed(attn, steps, warmup)
    b = W.decode_bytes(case.seq_lens, 8, 2, 256, 128)
    res = {"workload": "GQA paged decode, Qwen head shape 8q/2kv/256, 256 seqs, L log-uniform [128,32768]",
           "value": round(b["attention"] / ms / 1e6, 2), "unit": "GB/s", "ms_per_call": round(ms, 5),
           "roofline": {"bound": "hbm", "kernel": "paged_decode bf16 operator (head_dim 256)",
                        "achieved": round(b["attention"] / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(b["attention"] / ms / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms, 5), "algorithmic_bytes": b["attention"]}}
    del kc, vc
    torch.cuda.empty_cache()
    return res


def bench_decode_page16(seed, steps, warmup):
    """Config 2's sequences and heads over the reference's 16-token bf16 pages
    (native/include/paged_state_contract.h:25): 256 seqs, log-uniform
    [128, 32768], random block tables over a pool of 16-token pages."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    lens = W.decode_meta(seed, **W.CONFIGS["decode"]).seq_lens
    need = int(((lens.astype(np.int64) + 15) // 16).sum())
    kw = dict(W.CONFIGS["decode"])
    kw.update(block_size=16, pool_blocks=need + 64)
    case = W.decode_meta(seed, **kw)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 9)
    shape = (case.pool_blocks, 16, 2, 128)
    kc = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    fill_randn(kc, g)
    fill_randn(vc, g)
    q = torch.randn((256, 16, 128), generator=g, device=dev).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens_d = torch.from_numpy(case.seq_lens).to(dev)
    ws = ops.decode_workspace(256, 16, 128, case.max_context)
    out = torch.empty_like(q)

    def attn():
        ops.paged_decode(q, kc, vc, tables, lens_d, case.max_context, case.scale, out=out, workspace=ws)

    ms = timed(attn, steps, warmup)
    b = W.decode_bytes(case.seq_lens, 16, 2, 128, 16)["attention"]
    res = {"workload": "GQA paged decode on 16-token pages, config-2 sequences (256, log-uniform [128,32768])",
           "value": round(b / ms / 1e6, 2), "unit": "GB/s", "ms_per_call": round(ms, 5),
           "roofline": {"bound": "hbm", "kernel": "paged_decode bf16 operator (16-token pages)",
                        "achieved": round(b / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(b / ms / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms, 5), "algorithmic_bytes": b}}
    del kc, vc
    torch.cuda.empty_cache()
    return res


def bench_mla_c8(seed, steps, warmup):
    """Config 5's rows and lengths over packed C8 latent rows (656 B per key)."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    case = W.mla_meta(seed)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 6)
    n = case.pool_blocks * case.block_size
    cache = torch.empty((case.pool_blocks, case.block_size, 656), dtype=torch.uint8, device=dev)
    src = torch.empty((1 << 16, 576), dtype=torch.bfloat16, device=dev)
    for r0 in range(0, n, 1 << 16):
        fill_randn(src, g, std=0.5)
        m = min(1 << 16, n - r0)
        ops.mla_cache_write_c8(src[:m], cache, torch.arange(r0, r0 + m, dtype=torch.int64, device=dev))
    del src
    q = (torch.randn((case.num_seqs, case.heads, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens = torch.from_numpy(case.seq_lens).to(dev)
    ws = ops.mla_workspace(case.num_seqs, case.heads, case.max_context, case.block_size)
    out = torch.empty((case.num_seqs, case.heads, 512), dtype=torch.bfloat16, device=dev)

    def attn():
        ops.mla_decode(q, cache, tables, lens, case.max_context, case.scale, out=out, workspace=ws)

    ms = timed(attn, steps, warmup)
    L = case.seq_lens.astype(np.int64)
    nbytes = int(L.sum()) * 656 + case.num_seqs * case.heads * (576 + 512) * 2 + \
        int(((L + 63) // 64).sum()) * 4 + case.num_seqs * 4
    res = {"workload": "packed-MLA latent decode over C8 rows, config-5 rows and lengths",
           "value": round(nbytes / ms / 1e6, 2), "unit": "GB/s", "ms_per_call": round(ms, 5),
           "roofline": {"bound": "hbm", "kernel": "mla_decode c8 operator",
                        "achieved": round(nbytes / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms, 5), "algorithmic_bytes": nbytes}}
    del cache
    torch.cuda.empty_cache()
    return res


def bench_mla_rowq(seed, steps, warmup, bits):
    """Config 5's rows and lengths over row-quantized latent rows (the
    reference's integer cache: int8 or int4 codes of all 576 dims, one fp32
    scale per row), attended directly with in-register dequantization. Codes
    and scales are drawn at random (the kernel's cost does not depend on how
    they were produced)."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    case = W.mla_meta(seed)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 8 + bits)
    row_bytes = 576 * bits // 8
    cache = torch.randint(0, 256, (case.pool_blocks, case.block_size, row_bytes), generator=g,
                          device=dev, dtype=torch.uint8)
    scales = torch.rand(case.pool_blocks * case.block_size, generator=g, device=dev) * 0.01 + 0.001
    q = (torch.randn((case.num_seqs, case.heads, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens = torch.from_numpy(case.seq_lens).to(dev)
    n = ops.lib().ifattn_mla_attention_workspace_size(case.num_seqs, case.heads, case.max_context, 0, 0, 0,
                                                      case.block_size)
    ws = torch.empty(max(int(n), 16), dtype=torch.uint8, device=dev)
    out = torch.empty((case.num_seqs, case.heads, 512), dtype=torch.bfloat16, device=dev)

    def attn():
        ops.mla_attention(q, cache, tables, lens, case.max_context, scale=case.scale, out=out,
                          workspace=ws, row_scales=scales, bits=bits)

    ms = timed(attn, steps, warmup)
    L = case.seq_lens.astype(np.int64)
    nbytes = int(L.sum()) * (row_bytes + 4) + case.num_seqs * case.heads * (576 + 512) * 2 + \
        int(((L + 63) // 64).sum()) * 4 + case.num_seqs * 4
    res = {"workload": f"packed-MLA latent decode over row-quantized int{bits} rows (+ fp32 row "
                       f"scale), config-5 rows and lengths",
           "value": round(nbytes / ms / 1e6, 2), "unit": "GB/s", "ms_per_call": round(ms, 5),
           "roofline": {"bound": "hbm", "kernel": f"mla_attention rowq{bits} operator",
                        "achieved": round(nbytes / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms, 5), "algorithmic_bytes": nbytes}}
    del cache
    torch.cuda.empty_cache()
    return res


def bench_mla(seed, steps, warmup):
    """Config 5: packed-MLA latent decode, 128 seqs, L log-uniform [1024,65536],
    16 heads, 576-wide bf16 rows, block 64, N(0,0.5)."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    case = W.mla_meta(seed)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 5)
    cache = torch.empty((case.pool_blocks, case.block_size, 576), dtype=torch.bfloat16, device=dev)
    fill_randn(cache, g, std=0.5)
    q = (torch.randn((case.num_seqs, case.heads, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    rows = (torch.randn((case.num_seqs, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens = torch.from_numpy(case.seq_lens).to(dev)
    slots = torch.from_numpy(case.slot_mapping.astype(np.int64)).to(dev)
    ws = ops.mla_workspace(case.num_seqs, case.heads, case.max_context, case.block_size)
    out = torch.empty((case.num_seqs, case.heads, 512), dtype=torch.bfloat16, device=dev)

    def attn():
        ops.mla_decode(q, cache, tables, lens, case.max_context, case.scale, out=out, workspace=ws)

    def step():
        ops.kv_cache_write(rows, None, cache, None, slots)
        attn()

    ms_step = timed(step, steps, warmup)
    ms_attn = timed(attn, steps, warmup)
    L = case.seq_lens.astype(np.int64)
    attn_b = int(L.sum()) * 1152 + case.num_seqs * case.heads * (576 + 512) * 2 + \
        int(((L + 63) // 64).sum()) * 4 + case.num_seqs * 4
    total_b = attn_b + case.num_seqs * (1152 * 2 + 8)
    flops = int(L.sum()) * case.heads * (576 + 512) * 2
    res = {"workload": "packed-MLA latent decode, 128 seqs, L log-uniform [1024,65536] (BASELINE config 5)",
           "value": round(total_b / ms_step / 1e6, 2), "unit": "GB/s",
           "ms_per_step": round(ms_step, 5), "tokens_per_s": round(case.num_seqs / ms_step * 1e3, 1),
           "total_context_tokens": int(L.sum()), "tflops": round(flops / ms_attn / 1e9, 2),
           "roofline": {"bound": "hbm", "kernel": "mla_decode bf16 operator",
                        "achieved": round(attn_b / ms_attn / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(attn_b / ms_attn / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms_attn, 5), "algorithmic_bytes": attn_b}}
    del cache
    torch.cuda.empty_cache()
    return res


def mla_step_pair(case, seed, steps, warmup, graph=False):
    """ms of (fused, separate) decode steps over an MlaCase: each sequence's new
    latent row normalized, roped and written at its last position, then the
    decode. Fused: one ifattn_mla_decode_step; separate: the writer launch, then
    the decode launch."""
    import torch
    from ironpangu_amd import ops
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 5)
    n = case.num_seqs
    cache = torch.empty((case.pool_blocks, case.block_size, 576), dtype=torch.bfloat16, device=dev)
    fill_randn(cache, g, std=0.5)
    q = (torch.randn((n, case.heads, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    x = torch.randn((n, 576), generator=g, device=dev).to(torch.bfloat16)
    gamma = (torch.rand((512,), generator=g, device=dev) + 0.5).to(torch.bfloat16)
    ang = torch.rand((n, 32), generator=g, device=dev) * 6.28
    cos = torch.cat([ang.cos(), ang.cos()], 1).to(torch.bfloat16)
    sin = torch.cat([ang.sin(), ang.sin()], 1).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    lens = torch.from_numpy(case.seq_lens).to(dev)
    last = case.seq_lens.astype(np.int64) - 1
    slots = torch.from_numpy(case.block_tables[np.arange(n), last // case.block_size].astype(np.int64)
                             * case.block_size + last % case.block_size).to(dev)
    ws = ops.mla_workspace(n, case.heads, case.max_context, case.block_size)
    out = torch.empty((n, case.heads, 512), dtype=torch.bfloat16, device=dev)

    def fused():
        ops.mla_decode_step(q, x, gamma, cos, sin, cache, tables, lens, case.max_context,
                            scale=case.scale, out=out, workspace=ws)

    def separate():
        ops.mla_norm_rope_cache_write(x, gamma, cos, sin, cache, slots)
        ops.mla_decode(q, cache, tables, lens, case.max_context, case.scale, out=out, workspace=ws)

    ms = (timed(fused, steps, warmup, graph=graph), timed(separate, steps, warmup, graph=graph))
    del cache
    torch.cuda.empty_cache()
    return ms


def bench_mla_step(seed, steps, warmup):
    """Config 5 as a whole decode step (fused writer + decode in one launch,
    against the two launches), and the same comparison on a small batch
    replayed from a HIP graph, where the saved launch shows."""
    from ironpangu_amd import workloads as W
    case = W.mla_meta(seed)
    ms_fused, ms_sep = mla_step_pair(case, seed, steps, warmup)
    small = W.mla_meta(seed, num_seqs=16, lo=256, hi=4096)
    sm_fused, sm_sep = mla_step_pair(small, seed, max(steps, 50), warmup, graph=True)
    n = case.num_seqs
    L = case.seq_lens.astype(np.int64)
    nbytes = int(L.sum()) * 1152 + n * case.heads * (576 + 512) * 2 + int(((L + 63) // 64).sum()) * 4 + \
        n * 4 + n * (1152 + 256 + 1152) + 1024
    res = {"workload": "fused MLA decode step: cache writer (RMSNorm + RoPE) + latent decode, "
                       "config-5 rows and lengths (bf16 rows)",
           "value": round(nbytes / ms_fused / 1e6, 2), "unit": "GB/s",
           "ms_per_step": round(ms_fused, 5), "ms_separate_launches": round(ms_sep, 5),
           "small_batch": {"workload": "16 sequences of 256..4096 keys, graph replay",
                           "ms_fused": round(sm_fused, 5), "ms_separate_launches": round(sm_sep, 5)},
           "roofline": {"bound": "hbm", "kernel": "mla decode step operator (one launch: rows + attention; "
                                                  "merge)",
                        "achieved": round(nbytes / ms_fused / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(nbytes / ms_fused / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms_fused, 5), "algorithmic_bytes": nbytes}}
    return res


BF16_MFMA_PEAK_TFLOPS = 2500.0


def bench_mixed(seed, steps, warmup):
    """Config 3: 8 prefill chunks (U[64,2048] rows after U[0,8192] cached) +
    192 decode rows (U[256,16384]) in one packed varlen call."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    case = W.mixed_meta(seed)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 3)
    nb, bs, hkv, hd, hq = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim, case.q_heads
    kc = torch.empty((nb, bs, hkv, hd), dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    fill_randn(kc, g)
    fill_randn(vc, g)
    tq = int(case.cu_seqlens[-1])
    q = torch.randn((tq, hq, hd), generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn((tq, hkv, hd), generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn((tq, hkv, hd), generator=g, device=dev).to(torch.bfloat16)
    tables = torch.from_numpy(case.block_tables).to(dev)
    cu = torch.from_numpy(case.cu_seqlens).to(dev)
    kv = torch.from_numpy(case.kv_lens).to(dev)
    slots = torch.from_numpy(case.slot_mapping.astype(np.int64)).to(dev)
    ws = ops.prefill_workspace(len(case.q_lens), tq, hq, hd, case.max_kv_len)
    out = torch.empty_like(q)
    nchunk = int((case.q_lens > 1).sum())
    # prefill-only view: the chunk sequences alone
    cu_p = cu[: nchunk + 1].contiguous()
    tq_p = int(case.cu_seqlens[nchunk])
    ws_p = ops.prefill_workspace(nchunk, tq_p, hq, hd, case.max_kv_len)

    def attn():
        ops.varlen_prefill(q, kc, vc, tables, cu, kv, case.max_q_len, case.max_kv_len, case.scale,
                           out=out, workspace=ws)

    def prefill_only():
        ops.varlen_prefill(q[:tq_p], kc, vc, tables[:nchunk], cu_p, kv[:nchunk], case.max_q_len,
                           case.max_kv_len, case.scale, out=out[:tq_p], workspace=ws_p)

    def step():
        ops.kv_cache_write(kn, vn, kc, vc, slots)
        attn()

    ms_step = timed(step, steps, warmup)
    ms_pf = timed(prefill_only, steps, warmup)
    flops = 0
    kv_bytes = 0
    for s in range(len(case.q_lens)):
        L, K = int(case.q_lens[s]), int(case.kv_lens[s])
        vis = np.arange(K - L + 1, K + 1, dtype=np.int64)
        if L > 1:
            flops += int(vis.sum()) * hq * hd * 4
        kv_bytes += K * hkv * hd * 2 * 2
    ms_attn = timed(attn, steps, warmup)
    tf = flops / ms_pf / 1e9
    res = {"workload": "mixed chunked prefill + decode packed batch (BASELINE config 3)",
           "value": round(flops / ms_step / 1e9, 2), "unit": "TFLOP/s (prefill flops / step time)",
           "ms_per_step": round(ms_step, 5), "ms_attention": round(ms_attn, 5),
           "prefill_rows": tq_p, "decode_rows": int((case.q_lens == 1).sum()),
           "prefill_flops": flops, "kv_bytes": kv_bytes,
           "roofline": {"bound": "mfma", "kernel": "varlen_prefill (8 chunks, prefill kernel)",
                        "achieved": round(tf, 2), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "avg_ms": round(ms_pf, 5)}}
    del kc, vc
    torch.cuda.empty_cache()
    return res


def bench_mla_rows(seed, steps, warmup, sparse):
    """MLA attention over query rows with 128 learned sinks: 128 decode rows,
    contexts U[4096, 65536], 16 heads. BF16 rows over a 2048-token window
    (16-token pages), or packed C8 rows over top-2048 causal candidate lists
    (32-token pages) gathered at random."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    rng = np.random.default_rng(seed + 11)
    n, heads, topk, window = 128, 16, 2048, 2048
    bs = 32 if sparse else 16
    lens = rng.integers(4096, 65537, n).astype(np.int32)
    ctx = 65536
    if sparse:
        need = (lens.astype(np.int64) + bs - 1) // bs
        pool = int(need.sum())
        table = W.block_tables_for(rng, lens, bs, pool, ctx // bs)
    else:
        # ring of the last window + 1 pages per sequence (sliding_window_layout.h)
        from ironpangu_amd.host import WindowLayout
        lay = WindowLayout(ctx, window, 1, bs)
        pool = n * lay.physical_pages
        table = np.stack([lay.table(np.arange(lay.physical_pages) + s * lay.physical_pages)
                          for s in range(n)]).astype(np.int32)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 12)
    row = 656 if sparse else 1152  # bytes per key row
    if sparse:
        cache = torch.empty((pool, bs, 656), dtype=torch.uint8, device=dev)
        src = torch.empty((1 << 16, 576), dtype=torch.bfloat16, device=dev)
        for r0 in range(0, pool * bs, 1 << 16):
            fill_randn(src, g, std=0.5)
            m = min(1 << 16, pool * bs - r0)
            ops.mla_cache_write_c8(src[:m], cache, torch.arange(r0, r0 + m, dtype=torch.int64, device=dev))
        idx = torch.empty((n, topk), dtype=torch.int32, device=dev)
        for i in range(n):  # distinct random causal candidates
            idx[i] = torch.randperm(int(lens[i]), generator=g, device=dev)[:topk].to(torch.int32)
    else:
        cache = torch.empty((pool, bs, 576), dtype=torch.bfloat16, device=dev)
        fill_randn(cache, g, std=0.5)
        idx = None
    q = (torch.randn((n, heads, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    sk = (torch.randn((128, 576), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    sv = (torch.randn((128, 512), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    tables = torch.from_numpy(table).to(dev)
    kv = torch.from_numpy(lens).to(dev)
    out = torch.empty((n, heads, 512), dtype=torch.bfloat16, device=dev)
    nws = ops.lib().ifattn_mla_attention_workspace_size(n, heads, ctx, 0 if sparse else window,
                                                        topk if sparse else 0, 128, bs)
    ws = torch.empty(int(nws), dtype=torch.uint8, device=dev)

    def attn():
        ops.mla_attention(q, cache, tables, kv, ctx, indices=idx, window=0 if sparse else window,
                          sink_keys=sk, sink_values=sv, out=out, workspace=ws)

    ms = timed(attn, steps, warmup)
    keys = n * (topk if sparse else window)
    nbytes = keys * row + n * heads * (576 + 512) * 2 + 128 * (576 + 512) * 2 + \
        (keys * 4 if sparse else n * ((window + bs - 1) // bs + 1) * 4)
    name = ("C8 sparse top-2048 MLA attention + 128 sinks" if sparse
            else "BF16 window-2048 MLA attention (ring pages) + 128 sinks")
    res = {"workload": f"{name}, 128 decode rows, 16 heads", "value": round(nbytes / ms / 1e6, 2),
           "unit": "GB/s", "ms_per_call": round(ms, 5), "keys_per_call": keys,
           "roofline": {"bound": "hbm", "kernel": "mla_attention operator (plan, attention, merge)",
                        "achieved": round(nbytes / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms, 5), "algorithmic_bytes": nbytes}}
    del cache
    torch.cuda.empty_cache()
    return res


def bench_gated(seed, steps, warmup):
    """The reference session's Qwen-shape paged attention
    (inferfabric_acl_paged_attention_prepare: 8 q / 2 kv heads, head_dim 256,
    per-position int64 rows, fp32 additive mask, output gate) at its batch bound
    of 64 requests over a 32768-position table: live lengths log-uniform
    [128, 32768] (mask -inf beyond), rows drawn at random from a 2^20-row pool."""
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W
    rng = np.random.default_rng(seed + 21)
    batch, context, slots = 64, 32768, 1 << 20
    lens = W.lengths(rng, batch, 128, context, "loguniform")
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 22)
    keys = torch.empty((slots, 512), dtype=torch.bfloat16, device=dev)
    vals = torch.empty_like(keys)
    fill_randn(keys, g)
    fill_randn(vals, g)
    table = torch.randint(0, slots, (batch, context), generator=g, device=dev, dtype=torch.int64)
    pos = torch.arange(context, device=dev)[None, :]
    mask = torch.where(pos < torch.from_numpy(lens).to(dev)[:, None], 0.0, float("-inf")).to(torch.float32)
    q = torch.randn((batch, 8, 256), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((batch, 512), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((batch, 512), generator=g, device=dev).to(torch.bfloat16)
    gate = torch.sigmoid(torch.randn((batch, 8, 256), generator=g, device=dev)).to(torch.bfloat16)
    append = table[torch.arange(batch, device=dev), torch.from_numpy(lens - 1).to(dev)].contiguous()
    out = torch.empty_like(q)
    nws = ops.lib().ifattn_gated_paged_attention_workspace_size(batch, context)
    ws = torch.empty(max(int(nws), 16), dtype=torch.uint8, device=dev)

    def step():
        ops.gated_paged_attention(q, k, v, gate, keys, vals, append, table, mask, out=out, workspace=ws)

    ms = timed(step, steps, warmup)
    live = int(lens.sum())
    # K and V rows of every live position, the table and mask of every position,
    # q / gate / out, and the appended rows read and written.
    nbytes = live * 2048 + batch * context * 12 + batch * 8 * 256 * 2 * 3 + batch * 1024 * 2
    res = {"workload": "Qwen-shape gated paged attention (session ABI), 64 requests, 32768-position "
                       "table, live lengths log-uniform [128, 32768]",
           "value": round(nbytes / ms / 1e6, 2), "unit": "GB/s", "ms_per_call": round(ms, 5),
           "live_positions": live,
           "roofline": {"bound": "hbm", "kernel": "gated paged attention operator (plan + row append, decode, merge)",
                        "achieved": round(nbytes / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms, 5), "algorithmic_bytes": nbytes}}
    del keys, vals
    torch.cuda.empty_cache()
    return res


def bench_slot_reuse(seed, steps, warmup):
    """Slot reuse on a 2 GiB page field (20992-byte pages, the packed C8 MLA
    page): state copy of 1 GiB of pages from one resident to another (read +
    write) and the page reset (zeroing) of 1 GiB of owned spans."""
    import torch
    from ironpangu_amd import ops
    page = 32 * 656
    n_pages = (2 << 30) // page
    field = torch.zeros(n_pages * page, dtype=torch.uint8, device="cuda")
    half = n_pages // 2
    rng = np.random.default_rng(seed)
    src = rng.permutation(half)
    plan = np.stack([src * page, (half + np.arange(half)) * page, np.full(half, page)], 1)
    ranges = torch.from_numpy(plan.astype(np.int64)).cuda()
    from ironpangu_amd.host import page_spans
    spans = torch.from_numpy(np.array(page_spans(rng.permutation(n_pages)[:half].astype(np.int32),
                                                 page, n_pages * page), np.int64)).cuda()
    ms_copy = timed(lambda: ops.state_copy(field, ranges), steps, warmup)
    ms_reset = timed(lambda: ops.page_reset(field, spans), steps, warmup)
    copy_b = 2 * half * page
    reset_b = half * page
    res = {"workload": "state copy (1 GiB of 20992-byte pages) and page reset (1 GiB of spans)",
           "value": round(copy_b / ms_copy / 1e6, 2), "unit": "GB/s (copy, read + write)",
           "ms_copy": round(ms_copy, 5), "ms_reset": round(ms_reset, 5),
           "reset_gbps": round(reset_b / ms_reset / 1e6, 2),
           "roofline": {"bound": "hbm", "kernel": "state_span_kernel<copy>",
                        "achieved": round(copy_b / ms_copy / 1e6, 2), "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": round(copy_b / ms_copy / 1e6 / HBM_PEAK_GBPS, 4),
                        "avg_ms": round(ms_copy, 5), "algorithmic_bytes": copy_b}}
    del field
    torch.cuda.empty_cache()
    return res


def bench_norm_rope_write(seed, steps, warmup):
    """Fused MLA cache writer at the reference's batch bound: 4096 rows of 576
    bf16 -> packed C8 rows at random slots of a 65536-row cache."""
    import torch
    from ironpangu_amd import ops
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 13)
    rows = 4096
    x = torch.randn((rows, 576), generator=g, device="cuda").to(torch.bfloat16)
    gamma = torch.randn(512, generator=g, device="cuda").to(torch.bfloat16)
    cs = torch.randn((rows, 64), generator=g, device="cuda").to(torch.bfloat16)
    sn = torch.randn((rows, 64), generator=g, device="cuda").to(torch.bfloat16)
    cache = torch.zeros((2048, 32, 656), dtype=torch.uint8, device="cuda")
    slots = torch.randperm(65536, generator=g, device="cuda")[:rows]
    call = lambda: ops.mla_norm_rope_cache_write(x, gamma, cs, sn, cache, slots)
    ms_eager = timed(call, steps, warmup)
    # A decode step captures this call into its graph: per-call time of a graph
    # of 20 back-to-back calls (one graph launch amortised over 20 nodes), the
    # device time without the Python launch path.
    def twenty():
        for _ in range(20):
            call()
    ms = timed(twenty, max(steps // 10, 5), 2, graph=True) / 20
    nbytes = rows * (1152 + 2 * 128 + 8 + 656) + 1024
    return {"workload": "fused RMSNorm + rope + C8 MLA cache write, 4096 rows (HIP graph of 20 calls)",
            "value": round(rows / ms * 1e3, 1), "unit": "rows/s", "ms_per_call": round(ms, 5),
            "ms_per_call_eager": round(ms_eager, 5),
            "roofline": {"bound": "hbm", "kernel": "mla_norm_rope_write_kernel",
                         "achieved": round(nbytes / ms / 1e6, 2), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
                         "avg_ms": round(ms, 5), "algorithmic_bytes": nbytes,
                         "note": "latency-bound at this size (8.5 MB per call: one row per wave, "
                                 "every wave resident at once); ms_per_call_eager includes the "
                                 "Python launch path"}}


SECONDARY = {
    "c8_decode": bench_c8,
    "mla_decode": bench_mla,
    "mla_decode_c8": bench_mla_c8,
    "mla_decode_rowq8": lambda seed, steps, warmup: bench_mla_rowq(seed, steps, warmup, 8),
    "mla_decode_rowq4": lambda seed, steps, warmup: bench_mla_rowq(seed, steps, warmup, 4),
    "mla_decode_step": bench_mla_step,
    "gqa_decode_hd256": bench_decode_hd256,
    "gqa_decode_page16": bench_decode_page16,
    "mixed_prefill_decode": bench_mixed,
    "gated_attention_qwen": bench_gated,
    "mla_window_attention": lambda seed, steps, warmup: bench_mla_rows(seed, steps, warmup, False),
    "mla_sparse_attention": lambda seed, steps, warmup: bench_mla_rows(seed, steps, warmup, True),
    "slot_reuse": bench_slot_reuse,
    "norm_rope_write": bench_norm_rope_write,
}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU; --gpus must be 1 (each GPU box "
                                   "has a single MI355X, and the decode path shards by sequence "
                                   "with no cross-GPU exchange)"}))
        sys.exit(2)
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd import workloads as W

    if args.only:
        print(json.dumps({args.only: SECONDARY[args.only](args.seed, args.steps, args.warmup)}))
        return

    if args.calibrate_copy:
        # Known traffic for scaling rocprof FETCH_SIZE / WRITE_SIZE: each copy
        # reads and writes exactly 1 GiB.
        src = torch.ones(1 << 29, dtype=torch.int16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30,
                          "launches": 5}))
        return

    case, t = gpu_workload(args.seed)
    ws = ops.decode_workspace(case.num_seqs, case.q_heads, case.head_dim, case.max_context)
    out = torch.empty_like(t["q"])
    def step(ev=None):
        # Slot-mapped write of the 256 new K/V rows + ragged paged decode, as one
        # operator call (two kernel launches).
        stream = torch.cuda.current_stream()
        if ev is not None:
            ev[0].record(stream)
        ops.paged_decode_step(t["q"], t["k_new"], t["v_new"], t["k_cache"], t["v_cache"],
                              t["slots"], t["tables"], t["lens"], case.max_context, case.scale,
                              out=out, workspace=ws)
        if ev is not None:
            ev[1].record(stream)

    # Steps are issued back to back on one stream (eager). On this ROCm stack a
    # single-step HIP graph replay measured slower than eager launches, and the
    # host enqueues a step far faster than the GPU runs it.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # HIP events on the stream the kernels are launched on (torch's current
    # stream, which ops.* passes to the library), around the timed region.
    launch_stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(launch_stream)
    for _ in range(args.steps):
        step()
    end.record(launch_stream)
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / args.steps

    # Also each step bracketed by its own event pair (includes the event
    # packets between steps); reported beside the timed-region figure.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    attn_ms = [a.elapsed_time(b) for a, b in evs]
    attn_avg = float(np.mean(attn_ms))

    nbytes = W.decode_bytes(case.seq_lens, case.q_heads, case.kv_heads, case.head_dim,
                            case.block_size)
    value = nbytes["total"] / (ms_step * 1e-3) / 1e9
    achieved = value  # operator launches over the timed region, per step
    res = {
        "metric": "paged-decode attention GB/s (% of 8 TB/s HBM) + decode tokens/s, 256 ragged seqs",
        "value": round(value, 2),
        "unit": "GB/s",
        "timing": "back-to-back eager steps on one stream, HIP events",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 caches, random block tables)",
        "config": {"workload": "ragged_paged_decode_256 (BASELINE config 2)",
                   "num_seqs": case.num_seqs, "context": "log-uniform [128, 32768]",
                   "total_context_tokens": int(case.seq_lens.sum()),
                   "q_heads": case.q_heads, "kv_heads": case.kv_heads,
                   "head_dim": case.head_dim, "block_size": case.block_size,
                   "pool_blocks": case.pool_blocks, "parallelism": "none (1 GPU)"},
        "tokens_per_s": round(case.num_seqs / (ms_step * 1e-3), 1),
        # Per-step distribution: each step bracketed by its own event pair.
        "step_ms_median": round(float(np.median(attn_ms)), 5),
        "step_ms_p95": round(float(np.percentile(attn_ms, 95)), 5),
        "hbm_fraction": round(value / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": nbytes["total"],
        "roofline": {"bound": "hbm", "kernel": "paged_decode_step operator (prologue: plan + row writes; decode; split-K merge)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(),
                     "traffic_note": "HBM bytes per decode-kernel launch, rocprofv3 FETCH_SIZE x2.0 + "
                                     "WRITE_SIZE x1.0 (profiles/hbm_traffic_decode_kernels.md)",
                     "avg_ms": round(ms_step, 5),
                     "avg_ms_note": "HIP events on the launch stream around the timed steps / steps; "
                                    "the three kernels run back to back (rocprof: prologue + decode + merge)",
                     "isolated_step_ms": round(attn_avg, 5),
                     "algorithmic_bytes": nbytes["total"]},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args.seed, args.cpu_sample_seqs)
    if not args.no_secondary:
        del t
        torch.cuda.empty_cache()
        res["secondary"] = {name: fn(args.seed, args.steps, args.warmup)
                            for name, fn in SECONDARY.items()}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
