"""Shared test helpers: host<->device conversion of bf16 bit arrays and the
tolerance check used for floating-point parity (1e-2 abs + 1e-2 rel, the
bound stated for bf16 attention outputs)."""
from __future__ import annotations

import numpy as np

ATOL = 1e-2
RTOL = 1e-2


def to_dev(a, dtype=None):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def bf16_host(t) -> np.ndarray:
    """bf16 device tensor -> fp32 numpy."""
    import torch
    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def bits_host(t) -> np.ndarray:
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def assert_close(actual, expected, atol=ATOL, rtol=RTOL, what="output"):
    actual = np.asarray(actual, np.float32)
    expected = np.asarray(expected, np.float32)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    assert np.isfinite(actual).all(), f"{what}: non-finite values"
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} values out of tolerance; "
                             f"worst at {i}: got {actual[i]} expected {expected[i]}")
    return float(err.max()) if err.size else 0.0


def fill_randn(t, gen, std=1.0, clip=None):
    """Fill a device tensor with seeded N(0, std) draws (optionally clipped),
    converted to its dtype, in slabs that bound the fp32 temporary."""
    import torch
    flat = t.view(-1)
    step = 1 << 27
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        x = torch.randn(n, generator=gen, device=t.device, dtype=torch.float32) * std
        if clip is not None:
            x.clamp_(-clip, clip)
        flat[i:i + n] = x.to(t.dtype)


def compact_blocks(tables, lens, block_size):
    """Blocks a batch references, and its tables remapped onto a compact pool
    that holds only those blocks (so the host side copies back only what the
    attention reads). Returns (used block ids int64, remapped int32 tables)."""
    tables = np.asarray(tables)
    lens = np.asarray(lens, dtype=np.int64)
    need = (lens + block_size - 1) // block_size
    mask = np.arange(tables.shape[1])[None, :] < need[:, None]
    used = np.unique(tables[mask].astype(np.int64))
    remap = np.zeros(int(tables.max()) + 1, dtype=np.int64)
    remap[used] = np.arange(used.size)
    compact = np.where(mask, remap[tables], 0).astype(np.int32)
    return used, compact


def remap_slots(slots, used, block_size):
    """Physical token rows of the full pool -> rows of the compact pool."""
    slots = np.asarray(slots, dtype=np.int64)
    pos = np.searchsorted(used, slots // block_size)
    assert np.all(used[pos] == slots // block_size), "slot outside the referenced blocks"
    return pos * block_size + slots % block_size


def assert_rel_l2(actual, expected, bound=0.02, what="output"):
    """Relative L2 error per leading index (sequence or row) within `bound`,
    the acceptance rule of crates/inferfabric-cli/src/npu_probe/attention.rs:269.
    At long contexts the outputs shrink toward 0 and a 1e-2 absolute bound alone
    would accept a wrong sequence; this catches one."""
    a = np.asarray(actual, np.float64).reshape(len(actual), -1)
    e = np.asarray(expected, np.float64).reshape(len(expected), -1)
    num = np.sqrt(((a - e) ** 2).sum(1))
    den = np.sqrt((e ** 2).sum(1))
    rel = np.where(den > 0, num / np.maximum(den, 1e-30), num)
    bad = np.nonzero(rel > bound)[0]
    if bad.size:
        raise AssertionError(f"{what}: {bad.size} of {len(rel)} rows above relative L2 {bound}: "
                             f"rows {bad[:16].tolist()} rel {np.round(rel[bad[:16]], 4).tolist()}")
    return float(rel.max()) if rel.size else 0.0
