"""GPU parity for packed-MLA latent decode (bf16 and packed C8 rows) and for
packed varlen chunked prefill with decode rows, against the fp32 oracle
(bf16 outputs within 1e-2 abs + 1e-2 rel)."""
import numpy as np
import pytest

import oracle
from helpers import assert_close, bf16_host, bits_host, to_dev
from ironpangu_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("heads,c8,bs", [(16, False, 64), (16, True, 64), (6, False, 32),
                                         (6, True, 128), (16, False, 256), (16, True, 32)])
def test_mla_decode(heads, c8, bs):
    import torch
    from ironpangu_amd import ops
    case = W.mla_host_case(3, num_seqs=6, lo=1, hi=5000, dist="loguniform", heads=heads,
                           block_size=bs, fixed={0: 1, 1: 4096, 2: 31, 3: 2049})
    h = case.host
    nb, bs = case.pool_blocks, case.block_size
    pool = h["pool"].copy()
    oracle.kv_write(h["row_new"], pool, case.slot_mapping)
    slots = to_dev(case.slot_mapping.astype(np.int64))
    if c8:
        cache = torch.zeros((nb, bs, 656), dtype=torch.uint8, device="cuda")
        allslots = torch.arange(nb * bs, dtype=torch.int64, device="cuda")
        ops.mla_cache_write_c8(to_dev(h["pool"]), cache, allslots)
        ops.mla_cache_write_c8(to_dev(h["row_new"]), cache, slots)
        packed = oracle.mla_pack_c8(pool)
    else:
        cache = to_dev(h["pool"]).view(nb, bs, 576)
        ops.kv_cache_write(to_dev(h["row_new"]), None, cache, None, slots)
    out = ops.mla_decode(to_dev(h["q"]), cache, to_dev(case.block_tables),
                         to_dev(case.seq_lens), case.max_context, case.scale)
    torch.cuda.synchronize()
    if c8:
        assert np.array_equal(cache.cpu().numpy().reshape(-1, 656), packed), "C8 rows not bit-exact"
        exp = oracle.mla_decode(h["q"], packed, case.block_tables, case.seq_lens, heads, bs,
                                case.scale, c8=True)
    else:
        assert np.array_equal(bits_host(cache).reshape(-1, 576), pool), "latent rows not bit-exact"
        exp = oracle.mla_decode(h["q"], pool, case.block_tables, case.seq_lens, heads, bs,
                                case.scale)
    assert_close(bf16_host(out), exp)


def test_mla_decode_shares_slide_the_block_window():
    # 16-token pages: a lane window holds 64 block ids (1024 keys); four rows
    # of about 100000 keys give each persistent workgroup a share of about
    # 1560 keys, so the window slides inside a share.
    import torch
    from ironpangu_amd import ops
    case = W.mla_host_case(5, num_seqs=4, lo=1, hi=100000, dist="uniform", heads=16,
                           block_size=16, fixed={0: 100000, 1: 99999, 2: 98000, 3: 100000})
    h = case.host
    nb, bs = case.pool_blocks, case.block_size
    pool = h["pool"].copy()
    oracle.kv_write(h["row_new"], pool, case.slot_mapping)
    cache = to_dev(h["pool"]).view(nb, bs, 576)
    ops.kv_cache_write(to_dev(h["row_new"]), None, cache, None,
                       to_dev(case.slot_mapping.astype(np.int64)))
    out = ops.mla_decode(to_dev(h["q"]), cache, to_dev(case.block_tables),
                         to_dev(case.seq_lens), case.max_context, case.scale)
    torch.cuda.synchronize()
    exp = oracle.mla_decode(h["q"], pool, case.block_tables, case.seq_lens, 16, bs, case.scale)
    assert_close(bf16_host(out), exp)


def _prefill(case):
    import torch
    from ironpangu_amd import ops
    h = case.host
    nb, bs, hkv, hd = case.pool_blocks, case.block_size, case.kv_heads, case.head_dim
    kc = to_dev(h["k_pool"]).view(nb, bs, hkv, hd)
    vc = to_dev(h["v_pool"]).view(nb, bs, hkv, hd)
    ops.kv_cache_write(to_dev(h["k_new"]), to_dev(h["v_new"]), kc, vc,
                       to_dev(case.slot_mapping.astype(np.int64)))
    out = ops.varlen_prefill(to_dev(h["q"]), kc, vc, to_dev(case.block_tables),
                             to_dev(case.cu_seqlens), to_dev(case.kv_lens), case.max_q_len,
                             case.max_kv_len, case.scale)
    torch.cuda.synchronize()
    k_ref, v_ref = h["k_pool"].copy(), h["v_pool"].copy()
    oracle.kv_write(h["k_new"], k_ref, case.slot_mapping)
    oracle.kv_write(h["v_new"], v_ref, case.slot_mapping)
    exp = oracle.varlen_prefill(h["q"], k_ref, v_ref, case.block_tables, case.cu_seqlens,
                                case.kv_lens, case.q_heads, hkv, hd, bs, case.scale)
    return out, exp


@pytest.mark.parametrize("hq,hkv,hd,bs", [(16, 2, 128, 128), (16, 2, 128, 32), (8, 2, 256, 64),
                                          (8, 1, 64, 32), (16, 16, 128, 64)])
def test_varlen_prefill_mixed(hq, hkv, hd, bs):
    case = W.mixed_host_case(5, n_chunks=3, chunk_lo=2, chunk_hi=300, prior_lo=0, prior_hi=600,
                             n_decode=4, dec_lo=1, dec_hi=900, q_heads=hq, kv_heads=hkv,
                             head_dim=hd, block_size=bs)
    out, exp = _prefill(case)
    assert_close(bf16_host(out), exp)


def test_varlen_prefill_edges():
    # chunk lengths at tile edges, a chunk with no prior context, a 1-token chunk
    # (decode row), and a long prior context
    case = W.mixed_host_case(8, n_chunks=6, chunk_lo=31, chunk_hi=97, prior_lo=0, prior_hi=5000,
                             n_decode=2, dec_lo=3000, dec_hi=4100, q_heads=16, kv_heads=2,
                             head_dim=128, block_size=128)
    out, exp = _prefill(case)
    assert_close(bf16_host(out), exp)


def test_mla_decode_c8_q_range():
    """C8 latent scores run in fp16 with q rescaled per head by a power of two:
    heads with |q| far beyond fp16's range (2^17 times the usual values, softmax
    scale shrunk to match) and heads with |q| near 2^-21 must match the oracle."""
    import torch
    from ironpangu_amd import ops
    heads = 16
    case = W.mla_host_case(4, num_seqs=4, lo=1, hi=3000, dist="loguniform", heads=heads,
                           block_size=64, fixed={0: 2500, 1: 33})
    h = case.host
    nb, bs = case.pool_blocks, case.block_size
    pool = h["pool"].copy()
    oracle.kv_write(h["row_new"], pool, case.slot_mapping)
    qf = (h["q"].astype(np.uint32) << 16).view(np.float32).copy()
    qf[:, : heads // 2] *= np.float32(2.0 ** 17)
    qf[:, heads // 2:] *= np.float32(2.0 ** -20)
    q = (qf.view(np.uint32) >> 16).astype(np.uint16)  # power-of-two scaling: still exact bf16
    scale = case.scale * 2.0 ** -17
    cache = torch.zeros((nb, bs, 656), dtype=torch.uint8, device="cuda")
    ops.mla_cache_write_c8(to_dev(pool), cache, torch.arange(nb * bs, dtype=torch.int64, device="cuda"))
    out = ops.mla_decode(to_dev(q), cache, to_dev(case.block_tables), to_dev(case.seq_lens),
                         case.max_context, scale)
    torch.cuda.synchronize()
    exp = oracle.mla_decode(q, oracle.mla_pack_c8(pool), case.block_tables, case.seq_lens, heads,
                            bs, scale, c8=True)
    assert_close(bf16_host(out), exp)


def test_mla_decode_wide_layout():
    """Dense bf16 calls with at least 2^18 possible keys (rows x max_context)
    run the two-workgroup layout: 64 rows at max_context 40000 (tables padded
    to cover it), actual lengths up to 6000."""
    import torch
    from ironpangu_amd import ops
    case = W.mla_host_case(9, num_seqs=64, lo=1, hi=6000, dist="loguniform", heads=16,
                           block_size=64, fixed={0: 6000, 1: 1, 2: 3072, 3: 3073})
    h = case.host
    nb, bs = case.pool_blocks, case.block_size
    max_context = 40000
    assert 64 * max_context >= 1 << 18
    tables = np.zeros((64, (max_context + bs - 1) // bs), np.int32)
    tables[:, :case.block_tables.shape[1]] = case.block_tables
    cache = to_dev(h["pool"]).view(nb, bs, 576)
    out = ops.mla_decode(to_dev(h["q"]), cache, to_dev(tables), to_dev(case.seq_lens), max_context,
                         case.scale)
    torch.cuda.synchronize()
    exp = oracle.mla_decode(h["q"], h["pool"], case.block_tables, case.seq_lens, 16, bs, case.scale)
    assert_close(bf16_host(out), exp)
