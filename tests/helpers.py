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
