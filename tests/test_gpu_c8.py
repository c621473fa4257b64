"""GPU parity for the int8 paths: quantizing cache writes (bit-exact codes and
scales against the oracle), C8 paged decode (within 1e-2 of the fp32 oracle over
the dequantized cache), the packed 656-byte MLA row writer and the legacy
if_cache_quantize / if_cache_dequantize / if_packed_attention_metadata launchers."""
import math

import numpy as np
import pytest

import oracle
from helpers import assert_close, bf16_host, bits_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _quantize_pool_on_gpu(case):
    """Fill int8 pools by running the quantizing write over every pool row."""
    import torch
    from ironpangu_amd import ops
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc = torch.zeros((nb, bs, hkv, hd), dtype=torch.int8, device="cuda")
    vc = torch.zeros_like(kc)
    ks = torch.zeros((nb, bs, hkv), dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    all_slots = torch.arange(nb * bs, dtype=torch.int64, device="cuda")
    ops.kv_cache_write_c8(to_dev(h["k_pool"]), to_dev(h["v_pool"]), kc, vc, ks, vs, all_slots)
    return kc, vc, ks, vs


def test_c8_write_bit_exact():
    import torch
    from ironpangu_amd import ops
    case = W.decode_host_case(5, num_seqs=4, lo=40, hi=300, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=32, pool_blocks=48, c8=True)
    h = case.host
    # plant rounding ties and a zero row among the rows
    x = h["k_pool"].copy()
    ties = W.bf16_bits(np.array([127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 3.5, -126.5], np.float32))
    x[0, 0, :8] = ties
    x[0, 0, 8:] = 0
    x[1, 1, :] = 0
    h["k_pool"] = x
    kc, vc, ks, vs = _quantize_pool_on_gpu(case)
    torch.cuda.synchronize()
    codes, scales = oracle.quant_rows(x, case.head_dim, zero_scale=1.0)
    assert np.array_equal(kc.cpu().numpy().reshape(-1, case.head_dim), codes)
    assert np.array_equal(ks.cpu().numpy().reshape(-1), scales)
    # the planted row: scale 1, ties to even
    assert list(kc.cpu().numpy().reshape(-1, 128)[0, :8]) == [127, 0, 2, 2, 0, -2, 4, -126]
    assert ks.cpu().numpy().reshape(-1)[1 * 2 + 1] == 1.0  # zero row (slot 1, kv head 1) -> scale 1.0
    vcodes, vscales = oracle.quant_rows(h["v_pool"], case.head_dim)
    assert np.array_equal(vc.cpu().numpy().reshape(-1, case.head_dim), vcodes)
    assert np.array_equal(vs.cpu().numpy().reshape(-1), vscales)


@pytest.mark.parametrize("hd,bs", [(128, 128), (64, 32), (256, 64)])
def test_c8_decode(hd, bs):
    import torch
    from ironpangu_amd import ops
    case = W.decode_host_case(9, num_seqs=5, lo=1, hi=2300, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=hd, block_size=bs,
                              pool_blocks=5 * ((2300 + bs - 1) // bs) + 2, c8=True)
    kc, vc, ks, vs = _quantize_pool_on_gpu(case)
    out = ops.paged_decode(to_dev(case.host["q"]), kc, vc, to_dev(case.block_tables),
                           to_dev(case.seq_lens), case.max_context, case.scale,
                           k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    exp = oracle.paged_decode(case.host["q"], kc.cpu().numpy(), vc.cpu().numpy(),
                              case.block_tables, case.seq_lens, 16, 2, hd, bs, case.scale,
                              k_scale=ks.cpu().numpy(), v_scale=vs.cpu().numpy())
    assert_close(bf16_host(out), exp)


def test_c8_decode_many_partitions():
    # more than 16 split-K partitions (1536-token partitions for C8 caches)
    import torch
    from ironpangu_amd import ops
    case = W.decode_host_case(10, num_seqs=2, lo=1, hi=30000, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=128, pool_blocks=480, c8=True)
    case.seq_lens[:] = [30000, 24577]
    case.block_tables = W.block_tables_for(np.random.default_rng(9), case.seq_lens, 128, 480,
                                           case.block_tables.shape[1])
    kc, vc, ks, vs = _quantize_pool_on_gpu(case)
    out = ops.paged_decode(to_dev(case.host["q"]), kc, vc, to_dev(case.block_tables),
                           to_dev(case.seq_lens), case.max_context, case.scale,
                           k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    exp = oracle.paged_decode(case.host["q"], kc.cpu().numpy(), vc.cpu().numpy(),
                              case.block_tables, case.seq_lens, 16, 2, 128, 128, case.scale,
                              k_scale=ks.cpu().numpy(), v_scale=vs.cpu().numpy())
    assert_close(bf16_host(out), exp)


def test_mla_c8_write_bit_exact():
    import torch
    from ironpangu_amd import ops
    rng = np.random.default_rng(2)
    rows = W.bf16_randn(rng, (40, 576), std=0.5)
    rows[3, 128:256] = 0  # zero tile -> scale 0, codes 0
    rows[5, 0] = W.bf16_bits(np.array([3.0], np.float32))[0]
    cache = torch.full((4, 16, 656), 0xA5, dtype=torch.uint8, device="cuda")
    slots = np.array([(i * 37) % 64 for i in range(40)], np.int64)
    ops.mla_cache_write_c8(to_dev(rows), cache, to_dev(slots))
    torch.cuda.synchronize()
    got = cache.cpu().numpy().reshape(64, 656)
    exp = np.full((64, 656), 0xA5, np.uint8)
    exp[slots] = oracle.mla_pack_c8(rows)
    assert np.array_equal(got, exp)
    sc = exp[slots[3], 640:656].view(np.float32)
    assert sc[1] == 0.0 and not exp[slots[3], 128:256].any()


@pytest.mark.parametrize("bits", [8, 4])
def test_legacy_quantize_dequantize(bits):
    """if_cache_quantize / if_cache_dequantize with the reference probe's row
    x[j] = bf16((j % 61 - 30) / 13), width 576, rows {0, 1, 31, 511}
    (native/probes/cache_quantization_probe.cpp:17-27)."""
    import torch
    from ironpangu_amd import ops
    width, rows = 576, 512
    x = W.bf16_bits(((np.arange(width) % 61) - 30).astype(np.float32) / np.float32(13.0))
    packed = torch.full((rows * width * bits // 8,), 0xA5, dtype=torch.uint8, device="cuda")
    scales = torch.ones(rows, dtype=torch.float32, device="cuda")
    pos = torch.zeros(1, dtype=torch.int64, device="cuda")
    xin = to_dev(x)
    ref_packed, ref_scale = oracle.quant_legacy(x, bits)
    for row in (0, 1, 31, 511):
        pos.fill_(row)
        ops.cache_quantize(xin, packed, scales, pos, bits)
        torch.cuda.synchronize()
        p = packed.cpu().numpy().reshape(rows, -1)
        assert np.array_equal(p[row], ref_packed), f"row {row}"
        assert scales.cpu().numpy()[row] == np.float32(ref_scale)
    # reference probe expectation: scale = max/limit, q = round-half-away(x/scale)
    xf = W.bf16_to_f32(x)
    limit = 127 if bits == 8 else 7
    assert abs(ref_scale - np.abs(xf).max() / limit) <= 1e-6
    out = torch.zeros(rows * width, dtype=torch.bfloat16, device="cuda")
    pos.fill_(31)
    ops.cache_dequantize(packed, scales, out, pos, width, bits)
    torch.cuda.synchronize()
    exp = oracle.dequant_legacy(packed.cpu().numpy(), scales.cpu().numpy(), 31, width, bits)
    assert np.array_equal(bits_host(out), exp)


def test_packed_attention_metadata():
    import torch
    from ironpangu_amd import ops
    positions = torch.tensor([0, 31, 32, 511, 600], dtype=torch.int64, device="cuda")
    idx = torch.zeros(5 * 512, dtype=torch.int32, device="cuda")
    lens = torch.zeros(5, dtype=torch.int32, device="cuda")
    ops.packed_attention_metadata(positions, idx, lens, 512)
    torch.cuda.synchronize()
    i = idx.cpu().numpy().reshape(5, 512)
    for r, pos in enumerate([0, 31, 32, 511, 600]):
        exp = np.where(np.arange(512) <= pos, np.arange(512), -1)
        assert np.array_equal(i[r], exp)
    assert list(lens.cpu().numpy()) == [1, 32, 33, 512, 601]


@pytest.mark.parametrize("q_scale", [1e-4, 300.0, 3e4])
def test_c8_decode_q_range(q_scale):
    """C8 keys are scored with the fp16 MFMA (q scaled per head by a power of
    two into fp16 range, codes biased by 1152): q far from unit size, small
    enough that fp16 would lose it or large enough to overflow without the
    scale, still gives the oracle's output. Heads mix magnitudes (every other
    head 1/8 of the scale) so the per-head scale is exercised."""
    import torch
    from ironpangu_amd import ops
    print(f"c8 q range {q_scale}", flush=True)
    case = W.decode_host_case(12, num_seqs=6, lo=1, hi=1500, dist="uniform", q_heads=16,
                              kv_heads=2, head_dim=128, block_size=64,
                              pool_blocks=6 * 24 + 2, c8=True)
    kc, vc, ks, vs = _quantize_pool_on_gpu(case)
    qf = W.bf16_to_f32(case.host["q"]) * np.float32(q_scale / 64.0)
    qf[:, 1::2] *= np.float32(0.125)
    q = W.bf16_bits(qf)
    scale = 1.0 / (q_scale * 0.5)  # keeps the softmax neither flat nor one-hot
    out = ops.paged_decode(to_dev(q), kc, vc, to_dev(case.block_tables), to_dev(case.seq_lens),
                           case.max_context, scale, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    exp = oracle.paged_decode(q, kc.cpu().numpy(), vc.cpu().numpy(), case.block_tables,
                              case.seq_lens, 16, 2, 128, 64, scale,
                              k_scale=ks.cpu().numpy(), v_scale=vs.cpu().numpy())
    assert_close(bf16_host(out), exp)
