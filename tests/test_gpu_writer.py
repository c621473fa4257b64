"""GPU parity of the fused MLA cache writer (RMSNorm * gamma + half rope +
bf16 or packed C8 row) against the CPU oracle: bit-exact cache bytes, untouched
rows unchanged, skipped slots, the reference probe's fixtures
(native/probes/prefill_cache_writer_probe.cpp:14-27) and random inputs."""
import numpy as np
import pytest

import oracle
from helpers import to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu
f32 = np.float32


def _run(x, gamma, c, s, slots, packed, nslots, slot_dtype=np.int64, fill=0xA5):
    import torch
    from ironpangu_amd import ops
    stride = 656 if packed else 1152
    host = np.full((nslots, stride), fill, np.uint8)
    exp = oracle.mla_norm_rope_write(x, gamma, c, s, slots, host.copy(), packed)
    dev = torch.from_numpy(host.copy()).cuda()
    cache = dev.view(nslots // 32, 32, 656) if packed else dev.view(torch.bfloat16).view(nslots // 32, 32, 576)
    ops.mla_norm_rope_cache_write(to_dev(x).view(torch.bfloat16), to_dev(gamma).view(torch.bfloat16),
                                  to_dev(c).view(torch.bfloat16), to_dev(s).view(torch.bfloat16),
                                  cache, to_dev(slots.astype(slot_dtype)))
    torch.cuda.synchronize()
    got = dev.cpu().numpy()
    return got, exp


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("rows", [1, 17, 127, 4096])
def test_writer_probe_fixture(packed, rows):
    page = 32 if packed else 16
    logical = 4096 + np.arange(rows)
    d = np.arange(576)
    x = W.bf16_bits(((logical[:, None] * 7 + d[None, :] * 11) % 97 - 48).astype(f32)
                    * (1 + d // 128).astype(f32) / f32(128))
    slots = ((logical // page) * 37 % (8192 // page)) * page + logical % page
    gamma = W.bf16_bits(np.ones(512, f32))
    c = W.bf16_bits(np.full((rows, 64), 0.8, f32))
    s = W.bf16_bits(np.full((rows, 64), 0.6, f32))
    got, exp = _run(x, gamma, c, s, slots, packed, 8192)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("slot_dtype", [np.int32, np.int64])
def test_writer_random(packed, slot_dtype):
    rng = np.random.default_rng(11)
    rows = 300
    x = W.bf16_bits((rng.standard_normal((rows, 576)) * rng.uniform(0.01, 30, (rows, 1))).astype(f32))
    x[7, 256:384] = 0          # zero tile
    x[9, :512] = 0             # zero latent
    gamma = W.bf16_bits(rng.uniform(-2, 2, 512).astype(f32))
    c = W.bf16_bits(rng.uniform(-1, 1, (rows, 64)).astype(f32))
    s = W.bf16_bits(rng.uniform(-1, 1, (rows, 64)).astype(f32))
    slots = rng.permutation(2048)[:rows].astype(np.int64)
    slots[3], slots[4] = -1, 5000  # skipped
    got, exp = _run(x, gamma, c, s, slots, packed, 2048, slot_dtype)
    assert np.array_equal(got, exp)


def test_writer_rejects_bad_rows():
    import torch
    from ironpangu_amd import ops
    from ironpangu_amd._native import IfattnError
    x = torch.zeros((4097, 576), dtype=torch.bfloat16, device="cuda")
    cs = torch.zeros((4097, 64), dtype=torch.bfloat16, device="cuda")
    cache = torch.zeros((8, 32, 656), dtype=torch.uint8, device="cuda")
    g = torch.ones(512, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(IfattnError):
        ops.mla_norm_rope_cache_write(x, g, cs, cs, cache, torch.zeros(4097, dtype=torch.int64, device="cuda"))
