"""Pins for the fused MLA cache writer of the CPU oracle
(oracle_mla_norm_rope_write): the fixtures and acceptance rules of the
reference's own probe (native/probes/prefill_cache_writer_probe.cpp:14-61,
packed_cache_probe.cpp:24-45), restated in float64 here, plus a non-unit gamma
and the zero-tile rule (docs/packed-mla-cache.md:36-37)."""
import numpy as np
import pytest

import oracle
from ironpangu_amd import workloads as W

f32 = np.float32


def bf(x):
    return W.bf16_bits(np.asarray(x, np.float32))


def fp(b):
    return W.bf16_to_f32(b).astype(np.float64)


def probe_inputs(rows, start, page, capacity=8192):
    """Inputs of prefill_cache_writer_probe.cpp:14-27: x[d] = bf16(((l*7 + d*11) % 97 - 48)
    * (1 + d/128) / 128) for logical row l, slot ((l/page)*37 % (capacity/page))*page + l%page."""
    logical = start + np.arange(rows)
    d = np.arange(576)
    val = ((logical[:, None] * 7 + d[None, :] * 11) % 97 - 48).astype(f32)
    x = bf(val * (1 + d // 128).astype(f32) / f32(128))
    slots = ((logical // page) * 37 % (capacity // page)) * page + logical % page
    return x, slots.astype(np.int64)


def check_row(out_row, x_row, c_row, s_row, gamma, packed):
    """Acceptance rules of prefill_cache_writer_probe.cpp:38-61 in float64."""
    xv = fp(x_row)
    norm = 1.0 / np.sqrt((xv[:512] ** 2).sum() / 512 + 1e-5)
    y = xv[:512] * norm * fp(gamma)
    if packed:
        codes = out_row[:512].view(np.int8).astype(np.int64)
        scales = out_row[640:656].view(np.float32).astype(np.float64)
        for t in range(4):
            mx = np.abs(y[128 * t:128 * t + 128]).max()
            scale = mx / 127
            assert abs(scales[t] - scale) <= 1e-5 + 0.002 * scale
            exp = np.zeros(128) if scale == 0 else np.rint(y[128 * t:128 * t + 128] / scale)
            assert np.abs(codes[128 * t:128 * t + 128] - exp).max() <= 1
        rope = out_row[512:640].view(np.uint16)
    else:
        lat = fp(out_row[:1024].view(np.uint16))
        assert (np.abs(lat - y) <= 0.0078125 * np.maximum(1.0, np.abs(y))).all()
        rope = out_row[1024:1152].view(np.uint16)
    a = W.bf16_to_f32(x_row[512:576])
    b = W.bf16_to_f32(x_row[512 + (np.arange(64) + 32) % 64])
    nb = np.where(np.arange(64) < 32, -b, b).astype(f32)
    exp_rope = bf(a * W.bf16_to_f32(c_row) + nb * W.bf16_to_f32(s_row))  # fp32 products, fp32 sum
    assert np.array_equal(rope, exp_rope), "rope bits"


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("rows", [1, 2, 17, 127])
def test_writer_matches_reference_probe(packed, rows):
    page, capacity = (32 if packed else 16), 8192
    stride = 656 if packed else 1152
    cache = np.full((capacity, stride), 0xA5, np.uint8)
    gamma = bf(np.ones(512, f32))
    for start in (0, 4096):
        x, slots = probe_inputs(rows, start, page, capacity)
        c = bf(np.full((rows, 64), 0.8, f32))
        s = bf(np.full((rows, 64), 0.6, f32))
        before = cache.copy()
        oracle.mla_norm_rope_write(x, gamma, c, s, slots, cache, packed)
        touched = np.zeros(capacity, bool)
        touched[slots] = True
        assert np.array_equal(cache[~touched], before[~touched]), "unwritten rows changed"
        for r in range(rows):
            check_row(cache[slots[r]], x[r], c[r], s[r], gamma, packed)


@pytest.mark.parametrize("packed", [False, True])
def test_writer_gamma_and_zero_tile(packed):
    rng = np.random.default_rng(7)
    rows = 9
    x = bf(rng.standard_normal((rows, 576)).astype(f32))
    x[3, 128:256] = 0          # a zero tile (scale 0, codes 0 when packed)
    x[5, :512] = 0             # an all-zero latent: rstd = 1/sqrt(eps), outputs 0
    gamma = bf(rng.uniform(0.25, 2.0, 512).astype(f32))
    c = bf(rng.uniform(-1, 1, (rows, 64)).astype(f32))
    s = bf(rng.uniform(-1, 1, (rows, 64)).astype(f32))
    slots = np.array([5, 0, 9, 2, 7, 1, -1, 3, 12], np.int64)  # -1 and 12 (>= 12 slots) skipped
    stride = 656 if packed else 1152
    cache = np.zeros((12, stride), np.uint8)
    oracle.mla_norm_rope_write(x, gamma, c, s, slots, cache, packed)
    for r in range(rows):
        if 0 <= slots[r] < 12:
            check_row(cache[slots[r]], x[r], c[r], s[r], gamma, packed)
    if packed:
        row = cache[slots[3]]
        assert row[640 + 4:640 + 8].view(np.float32)[0] == 0 and not row[128:256].any()
        assert not cache[slots[5]][:512].any()
    # an identity-gamma run differs wherever gamma != 1 (gamma is applied)
    cache1 = np.zeros_like(cache)
    oracle.mla_norm_rope_write(x, bf(np.ones(512, f32)), c, s, slots, cache1, packed)
    assert not np.array_equal(cache1[slots[0]], cache[slots[0]])
