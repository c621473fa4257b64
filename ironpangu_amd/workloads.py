"""Seeded synthetic workloads for the five benchmark configurations.

Generator: numpy ``default_rng(seed)`` (PCG64) for all metadata (lengths,
block tables, slot mappings) and for small host-side tensors; large cache
pools for the benchmark are drawn on the GPU with a seeded ``torch.Generator``.
Normal draws are rounded to bf16 with round-to-nearest-even.

Sequence convention: a decode sequence of context length L holds L tokens
after this step's append; the new token sits at position L-1 and its K/V rows
are written through the slot mapping before attention reads them (the order
of native/src/inferfabric_acl.cpp:1364-1428).

Configurations (BASELINE.json ``configs``):
  1 ``cpu_ref``  8 seqs, L ~ U[16,512], 16q/2kv/128, block 128, 512-block pool
  2 ``decode``   256 seqs, L log-uniform [128,32768], 16q/2kv/128, block 128, 65536-block pool
  3 ``mixed``    8 chunks of U[64,2048] rows after U[0,8192] cached + 192 decode rows L~U[256,16384]
  4 ``c8``       256 seqs, L ~ U[1024,16384], int8 K/V (N(0,1) clipped to +-4), fp32 scale/token/head
  5 ``mla``      128 seqs, L log-uniform [1024,65536], 16 heads, 576-wide rows, block 64, N(0,0.5)
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


# ------------------------------------------------------------------ bf16 helpers

def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round-to-nearest-even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_randn(rng, shape, std=1.0, clip=None) -> np.ndarray:
    x = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
    if clip is not None:
        x = np.clip(x, -clip, clip)
    return bf16_bits(x)


# ------------------------------------------------------------------ metadata

def lengths(rng, n, lo, hi, dist="uniform") -> np.ndarray:
    if dist == "uniform":
        return rng.integers(lo, hi + 1, size=n).astype(np.int32)
    if dist == "loguniform":
        x = np.exp(rng.uniform(math.log(lo), math.log(hi), size=n))
        return np.clip(np.rint(x), lo, hi).astype(np.int32)
    raise ValueError(dist)


def block_tables_for(rng, lens, block_size, pool_blocks, stride=None) -> np.ndarray:
    """Disjoint per-sequence block lists drawn from a random permutation of the pool."""
    need = (np.asarray(lens, dtype=np.int64) + block_size - 1) // block_size
    if int(need.sum()) > pool_blocks:
        raise ValueError("pool too small for the drawn lengths")
    stride = int(stride or max(1, int(need.max())))
    perm = rng.permutation(pool_blocks).astype(np.int32)
    table = np.zeros((len(lens), stride), dtype=np.int32)
    off = 0
    for i, k in enumerate(need):
        table[i, :k] = perm[off:off + k]
        off += int(k)
    return table


def slots_of(table, positions, seq_ids, block_size) -> np.ndarray:
    """Physical token row of each (sequence, position): table[p/bs]*bs + p%bs."""
    positions = np.asarray(positions, dtype=np.int64)
    blk = table[np.asarray(seq_ids), positions // block_size].astype(np.int64)
    return blk * block_size + positions % block_size


# ------------------------------------------------------------------ case objects

@dataclass
class DecodeCase:
    num_seqs: int
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    pool_blocks: int
    seq_lens: np.ndarray      # int32 [n]
    block_tables: np.ndarray  # int32 [n, stride]
    slot_mapping: np.ndarray  # int64 [n] slot of the new token (position L-1)
    max_context: int
    scale: float
    c8: bool = False
    host: dict = field(default_factory=dict)  # numpy payloads for small cases


CONFIGS = {
    "cpu_ref": dict(num_seqs=8, lo=16, hi=512, dist="uniform", q_heads=16, kv_heads=2,
                    head_dim=128, block_size=128, pool_blocks=512),
    "decode": dict(num_seqs=256, lo=128, hi=32768, dist="loguniform", q_heads=16, kv_heads=2,
                   head_dim=128, block_size=128, pool_blocks=65536),
    "c8": dict(num_seqs=256, lo=1024, hi=16384, dist="uniform", q_heads=16, kv_heads=2,
               head_dim=128, block_size=128, pool_blocks=32768),
}


def decode_meta(seed, num_seqs, lo, hi, dist, q_heads, kv_heads, head_dim, block_size,
                pool_blocks, c8=False, max_context=None) -> DecodeCase:
    rng = np.random.default_rng(seed)
    lens = lengths(rng, num_seqs, lo, hi, dist)
    max_context = int(max_context or hi)
    stride = (max_context + block_size - 1) // block_size
    table = block_tables_for(rng, lens, block_size, pool_blocks, stride)
    slots = slots_of(table, lens - 1, np.arange(num_seqs), block_size)
    return DecodeCase(num_seqs, q_heads, kv_heads, head_dim, block_size, pool_blocks, lens, table,
                      slots, max_context, 1.0 / math.sqrt(head_dim), c8)


def decode_host_case(seed, **kw) -> DecodeCase:
    """Small case with every tensor materialised on the host (numpy)."""
    c = decode_meta(seed, **kw)
    rng = np.random.default_rng(seed + 1)
    nslot = c.pool_blocks * c.block_size
    clip = 4.0 if c.c8 else None
    c.host["q"] = bf16_randn(rng, (c.num_seqs, c.q_heads, c.head_dim))
    c.host["k_new"] = bf16_randn(rng, (c.num_seqs, c.kv_heads, c.head_dim), clip=clip)
    c.host["v_new"] = bf16_randn(rng, (c.num_seqs, c.kv_heads, c.head_dim), clip=clip)
    c.host["k_pool"] = bf16_randn(rng, (nslot, c.kv_heads, c.head_dim), clip=clip)
    c.host["v_pool"] = bf16_randn(rng, (nslot, c.kv_heads, c.head_dim), clip=clip)
    return c


def config_case(name, seed=0, host=True) -> DecodeCase:
    kw = dict(CONFIGS[name])
    kw["c8"] = name == "c8"
    return decode_host_case(seed, **kw) if host else decode_meta(seed, **kw)


# ------------------------------------------------------------------ mixed prefill

@dataclass
class MixedCase:
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    pool_blocks: int
    q_lens: np.ndarray        # rows per sequence (chunk length, 1 for decode rows)
    kv_lens: np.ndarray       # cached context after this step's writes
    cu_seqlens: np.ndarray    # int32 [n+1]
    block_tables: np.ndarray
    slot_mapping: np.ndarray  # int64 [total_q] slots of every new row
    max_q_len: int
    max_kv_len: int
    scale: float
    host: dict = field(default_factory=dict)


def mixed_meta(seed=0, n_chunks=8, chunk_lo=64, chunk_hi=2048, prior_lo=0, prior_hi=8192,
               n_decode=192, dec_lo=256, dec_hi=16384, q_heads=16, kv_heads=2, head_dim=128,
               block_size=128, pool_blocks=None) -> MixedCase:
    rng = np.random.default_rng(seed)
    chunk = lengths(rng, n_chunks, chunk_lo, chunk_hi)
    prior = lengths(rng, n_chunks, prior_lo, prior_hi)
    dec = lengths(rng, n_decode, dec_lo, dec_hi)
    q_lens = np.concatenate([chunk, np.ones(n_decode, np.int32)]).astype(np.int32)
    kv_lens = np.concatenate([prior + chunk, dec]).astype(np.int32)
    max_kv = int(max(prior_hi + chunk_hi, dec_hi))
    stride = (max_kv + block_size - 1) // block_size
    need = int(((kv_lens.astype(np.int64) + block_size - 1) // block_size).sum())
    pool = int(pool_blocks or need + 64)
    table = block_tables_for(rng, kv_lens, block_size, pool, stride)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    seq_of_row = np.repeat(np.arange(len(q_lens)), q_lens)
    pos = np.concatenate([np.arange(kv - q, kv) for q, kv in zip(q_lens, kv_lens)])
    slots = slots_of(table, pos, seq_of_row, block_size)
    return MixedCase(q_heads, kv_heads, head_dim, block_size, pool, q_lens, kv_lens, cu, table,
                     slots, int(q_lens.max()), max_kv, 1.0 / math.sqrt(head_dim))


def mixed_host_case(seed=0, **kw) -> MixedCase:
    c = mixed_meta(seed, **kw)
    rng = np.random.default_rng(seed + 1)
    tq = int(c.cu_seqlens[-1])
    nslot = c.pool_blocks * c.block_size
    c.host["q"] = bf16_randn(rng, (tq, c.q_heads, c.head_dim))
    c.host["k_new"] = bf16_randn(rng, (tq, c.kv_heads, c.head_dim))
    c.host["v_new"] = bf16_randn(rng, (tq, c.kv_heads, c.head_dim))
    c.host["k_pool"] = bf16_randn(rng, (nslot, c.kv_heads, c.head_dim))
    c.host["v_pool"] = bf16_randn(rng, (nslot, c.kv_heads, c.head_dim))
    return c


# ------------------------------------------------------------------ MLA

@dataclass
class MlaCase:
    num_seqs: int
    heads: int
    block_size: int
    pool_blocks: int
    seq_lens: np.ndarray
    block_tables: np.ndarray
    slot_mapping: np.ndarray
    max_context: int
    scale: float
    c8: bool = False
    host: dict = field(default_factory=dict)


def mla_meta(seed=0, num_seqs=128, lo=1024, hi=65536, dist="loguniform", heads=16, block_size=64,
             pool_blocks=None, c8=False, fixed=None) -> MlaCase:
    """``fixed`` maps sequence index -> length, overriding the drawn ones."""
    rng = np.random.default_rng(seed)
    lens = lengths(rng, num_seqs, lo, hi, dist)
    for i, n in (fixed or {}).items():
        lens[i] = n
    stride = (hi + block_size - 1) // block_size
    need = int(((lens.astype(np.int64) + block_size - 1) // block_size).sum())
    pool = int(pool_blocks or need + 64)
    table = block_tables_for(rng, lens, block_size, pool, stride)
    slots = slots_of(table, lens - 1, np.arange(num_seqs), block_size)
    return MlaCase(num_seqs, heads, block_size, pool, lens, table, slots, hi,
                   1.0 / math.sqrt(192.0), c8)


def mla_host_case(seed=0, **kw) -> MlaCase:
    c = mla_meta(seed, **kw)
    rng = np.random.default_rng(seed + 1)
    nslot = c.pool_blocks * c.block_size
    c.host["q"] = bf16_randn(rng, (c.num_seqs, c.heads, 576), std=0.5)
    c.host["row_new"] = bf16_randn(rng, (c.num_seqs, 576), std=0.5)
    c.host["pool"] = bf16_randn(rng, (nslot, 576), std=0.5)
    return c


# ------------------------------------------------------------------ algorithmic bytes

def decode_bytes(lens, q_heads, kv_heads, head_dim, block_size, elem_bytes=2, scale_bytes=0,
                 with_write=True) -> dict:
    """Bytes that must cross HBM once for one decode step (K/V rows over the
    visible context, q in, out, block-table entries, and the new rows'
    read + write)."""
    lens = np.asarray(lens, dtype=np.int64)
    n = len(lens)
    kv_row = kv_heads * (head_dim * elem_bytes + scale_bytes)
    attn = int(lens.sum()) * 2 * kv_row + n * q_heads * head_dim * 2 * 2 + \
        int(((lens + block_size - 1) // block_size).sum()) * 4 + n * 4
    write = n * 2 * (kv_heads * head_dim * 2 + kv_row) + n * 8 if with_write else 0
    return {"attention": attn, "write": write, "total": attn + write}
