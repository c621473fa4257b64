"""Torch-tensor wrappers over the C ABI (device memory and streams come from
torch; every kernel is the native gfx950 code in ``libifattn_hip.so``).

Shapes are validated on the host before any launch so that a kernel never
runs on operands that disagree with its grid. Each call is asynchronous on
torch's current stream (or ``stream`` when given).

Cache layouts (see include/ifattn.h):
  GQA K/V cache  [num_blocks, block_size, kv_heads, head_dim]   bf16 or int8
  C8 scales      [num_blocks, block_size, kv_heads]             fp32
  MLA cache      [num_blocks, block_size, 576] bf16 or [num_blocks, block_size, 656] uint8
"""
from __future__ import annotations

import math

import torch

from ._native import check, lib

I32, I64 = 4, 5


def _stream(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _req(cond, msg):
    if not cond:
        raise ValueError(msg)


def _dev(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        _req(t.is_cuda, "all tensors must be on the GPU")
        _req(t.is_contiguous(), "all tensors must be contiguous")
        dev = dev or t.device
        _req(t.device == dev, "all tensors must be on one device")


def _slot_dtype(slots):
    _req(slots.dtype in (torch.int32, torch.int64), "slot_mapping must be int32 or int64")
    return I32 if slots.dtype == torch.int32 else I64


# ---------------------------------------------------------------- cache writes

def kv_cache_write(k, v, k_cache, v_cache, slot_mapping, stream=None):
    """cache[slot_mapping[r]] = rows[r] (bit copy) for K and, if given, V.

    k, v: [rows, ...]; caches: [num_blocks, block_size, ...] with the same
    per-token row; slot_mapping: [rows] int32/int64 physical token rows.
    """
    _dev(k, v, k_cache, v_cache, slot_mapping)
    rows = k.shape[0]
    row_bytes = k[0].numel() * k.element_size() if rows else 0
    _req(slot_mapping.numel() == rows, "one slot per row")
    _req(k_cache.dtype == k.dtype, "row and cache dtypes differ")
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    _req(k_cache.numel() * k_cache.element_size() == num_slots * row_bytes or rows == 0,
         "cache row width differs from input row width")
    if v is not None:
        _req(v.shape == k.shape and v_cache.shape == k_cache.shape, "K/V shapes differ")
    check(lib().ifattn_kv_cache_write(_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                      _ptr(slot_mapping), _slot_dtype(slot_mapping), rows,
                                      max(row_bytes, 16), num_slots, _stream(stream)),
          "ifattn_kv_cache_write")


def kv_cache_write_c8(k, v, k_cache, v_cache, k_scale, v_scale, slot_mapping, stream=None):
    """Quantizing write: bf16 [rows, kv_heads, head_dim] -> int8 caches
    [blocks, block_size, kv_heads, head_dim] and fp32 scales [blocks, block_size, kv_heads]."""
    _dev(k, v, k_cache, v_cache, k_scale, v_scale, slot_mapping)
    _req(k.dtype == torch.bfloat16 and k.dim() == 3, "k rows: bf16 [rows, kv_heads, head_dim]")
    rows, kvh, hd = k.shape
    _req(k_cache.dtype == torch.int8 and k_cache.dim() == 4 and tuple(k_cache.shape[2:]) == (kvh, hd),
         "k cache: int8 [blocks, block_size, kv_heads, head_dim]")
    _req(k_scale.dtype == torch.float32 and tuple(k_scale.shape) == tuple(k_cache.shape[:3]),
         "k scale: fp32 [blocks, block_size, kv_heads]")
    if v is not None:
        _req(v.shape == k.shape and v_cache.shape == k_cache.shape and v_scale.shape == k_scale.shape,
             "K/V shapes differ")
    _req(slot_mapping.numel() == rows, "one slot per row")
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    check(lib().ifattn_kv_cache_write_c8(_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                         _ptr(k_scale), _ptr(v_scale), _ptr(slot_mapping),
                                         _slot_dtype(slot_mapping), rows, kvh, hd, num_slots,
                                         _stream(stream)),
          "ifattn_kv_cache_write_c8")


def mla_cache_write_c8(rows, cache, slot_mapping, stream=None):
    """bf16 [rows, 576] -> packed 656-byte rows of a uint8 [blocks, block_size, 656] cache."""
    _dev(rows, cache, slot_mapping)
    _req(rows.dtype == torch.bfloat16 and rows.dim() == 2 and rows.shape[1] == 576,
         "rows: bf16 [rows, 576]")
    _req(cache.dtype == torch.uint8 and cache.dim() == 3 and cache.shape[2] == 656,
         "cache: uint8 [blocks, block_size, 656]")
    _req(slot_mapping.numel() == rows.shape[0], "one slot per row")
    check(lib().ifattn_mla_cache_write_c8(_ptr(rows), _ptr(cache), _ptr(slot_mapping),
                                          _slot_dtype(slot_mapping), rows.shape[0],
                                          cache.shape[0] * cache.shape[1], _stream(stream)),
          "ifattn_mla_cache_write_c8")


def mla_norm_rope_cache_write(x, gamma, cos, sin, cache, slot_mapping, eps=1e-5, stream=None):
    """Fused RMSNorm(512) * gamma + half rotary(64) + cache store of bf16 x [rows, 576].

    cache: bf16 [blocks, block_size, 576] (bf16 rows) or uint8 [blocks, block_size, 656]
    (packed C8 rows); gamma [512] bf16; cos/sin [rows, 64] bf16; rows 1..4096.
    """
    _dev(x, gamma, cos, sin, cache, slot_mapping)
    _req(x.dtype == torch.bfloat16 and x.dim() == 2 and x.shape[1] == 576, "x: bf16 [rows, 576]")
    rows = x.shape[0]
    _req(gamma.dtype == torch.bfloat16 and gamma.numel() == 512, "gamma: bf16 [512]")
    for t, n in ((cos, "cos"), (sin, "sin")):
        _req(t.dtype == torch.bfloat16 and tuple(t.shape) == (rows, 64), f"{n}: bf16 [rows, 64]")
    _req(cache.dim() == 3, "cache: [blocks, block_size, row]")
    if cache.dtype == torch.uint8:
        _req(cache.shape[2] == 656, "packed cache rows are 656 bytes")
        packed = 1
    else:
        _req(cache.dtype == torch.bfloat16 and cache.shape[2] == 576, "bf16 cache rows are 576 wide")
        packed = 0
    _req(slot_mapping.numel() == rows, "one slot per row")
    check(lib().ifattn_mla_norm_rope_cache_write(_ptr(x), _ptr(gamma), _ptr(cos), _ptr(sin),
                                                 _ptr(slot_mapping), _slot_dtype(slot_mapping),
                                                 rows, float(eps), _ptr(cache), packed,
                                                 cache.shape[0] * cache.shape[1], _stream(stream)),
          "ifattn_mla_norm_rope_cache_write")


# ---------------------------------------------------------------- decode

def decode_workspace(num_seqs, q_heads, head_dim, max_context, device="cuda"):
    n = lib().ifattn_paged_decode_workspace_size(num_seqs, q_heads, head_dim, max_context)
    return torch.empty(max(int(n), 16), dtype=torch.uint8, device=device)


def _check_tables(block_tables, seq_lens, num_seqs, block_size, max_context):
    _req(block_tables.dtype == torch.int32 and block_tables.dim() == 2
         and block_tables.shape[0] >= num_seqs, "block_tables: int32 [num_seqs, entries]")
    _req(block_tables.shape[1] * block_size >= max_context,
         "block_tables do not cover max_context")
    _req(seq_lens.dtype == torch.int32 and seq_lens.numel() >= num_seqs, "seq_lens: int32 [num_seqs]")


def paged_decode(q, k_cache, v_cache, block_tables, seq_lens, max_context, scale=None,
                 out=None, workspace=None, k_scale=None, v_scale=None, stream=None):
    """Ragged paged GQA decode. q [num_seqs, q_heads, head_dim] bf16.

    bf16 caches, or int8 caches with fp32 k_scale/v_scale. Returns out
    [num_seqs, q_heads, head_dim] bf16.
    """
    c8 = k_cache.dtype == torch.int8
    _dev(q, k_cache, v_cache, block_tables, seq_lens, out, workspace, k_scale, v_scale)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3, "q: bf16 [num_seqs, q_heads, head_dim]")
    ns, hq, hd = q.shape
    _req(k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.shape[3] == hd,
         "caches: [num_blocks, block_size, kv_heads, head_dim]")
    nb, bs, hkv, _ = k_cache.shape
    _req(k_cache.dtype == (torch.int8 if c8 else torch.bfloat16) and v_cache.dtype == k_cache.dtype,
         "cache dtype must be bf16 or int8 (both caches)")
    if c8:
        _req(k_scale is not None and v_scale is not None and k_scale.dtype == torch.float32
             and tuple(k_scale.shape) == (nb, bs, hkv) and v_scale.shape == k_scale.shape,
             "int8 caches need fp32 scales [num_blocks, block_size, kv_heads]")
    _check_tables(block_tables, seq_lens, ns, bs, max_context)
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    if out is None:
        out = torch.empty_like(q)
    _req(out.shape == q.shape and out.dtype == torch.bfloat16, "out: bf16 like q")
    if workspace is None:
        workspace = decode_workspace(ns, hq, hd, max_context, q.device)
    stride = block_tables.shape[1]
    if c8:
        st = lib().ifattn_paged_decode_c8(
            _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
            _ptr(block_tables), stride, _ptr(seq_lens), _ptr(out), ns, hq, hkv, hd, bs, nb,
            max_context, float(scale), _ptr(workspace), workspace.numel(), _stream(stream))
        check(st, "ifattn_paged_decode_c8")
    else:
        st = lib().ifattn_paged_decode_bf16(
            _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), stride, _ptr(seq_lens),
            _ptr(out), ns, hq, hkv, hd, bs, nb, max_context, float(scale), _ptr(workspace),
            workspace.numel(), _stream(stream))
        check(st, "ifattn_paged_decode_bf16")
    return out


def paged_decode_step(q, k_new, v_new, k_cache, v_cache, slot_mapping, block_tables, seq_lens,
                      max_context, scale=None, out=None, workspace=None, stream=None):
    """Slot-mapped write of k_new/v_new [rows, kv_heads, head_dim] followed by
    paged decode over the updated bf16 caches, in two launches."""
    _dev(q, k_new, v_new, k_cache, v_cache, slot_mapping, block_tables, seq_lens, out, workspace)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3, "q: bf16 [num_seqs, q_heads, head_dim]")
    ns, hq, hd = q.shape
    _req(k_cache.dtype == torch.bfloat16 and k_cache.dim() == 4 and k_cache.shape == v_cache.shape
         and k_cache.shape[3] == hd, "caches: bf16 [num_blocks, block_size, kv_heads, head_dim]")
    nb, bs, hkv, _ = k_cache.shape
    _req(k_new.shape == v_new.shape and k_new.dim() == 3 and tuple(k_new.shape[1:]) == (hkv, hd)
         and k_new.dtype == torch.bfloat16, "new rows: bf16 [rows, kv_heads, head_dim]")
    _req(slot_mapping.numel() == k_new.shape[0], "one slot per new row")
    _check_tables(block_tables, seq_lens, ns, bs, max_context)
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = decode_workspace(ns, hq, hd, max_context, q.device)
    st = lib().ifattn_paged_decode_step_bf16(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping),
        _slot_dtype(slot_mapping), k_new.shape[0], _ptr(block_tables), block_tables.shape[1],
        _ptr(seq_lens), _ptr(out), ns, hq, hkv, hd, bs, nb, max_context, float(scale),
        _ptr(workspace), workspace.numel(), _stream(stream))
    check(st, "ifattn_paged_decode_step_bf16")
    return out


def gated_paged_attention(q, k, v, gate, keys, values, append, table, mask, out=None,
                          workspace=None, stream=None):
    """Qwen-shape session attention (inferfabric_acl_paged_attention_prepare):
    append k/v [batch, 512] at keys/values[append], then attend q [batch, 8, 256]
    over the per-position rows ``table`` [batch, context] int64 with the fp32
    additive ``mask`` [batch, context], times ``gate`` [batch, 8, 256]."""
    _dev(q, k, v, gate, keys, values, append, table, mask, out, workspace)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3 and tuple(q.shape[1:]) == (8, 256),
         "q: bf16 [batch, 8, 256]")
    batch = q.shape[0]
    for t, n in ((k, "k"), (v, "v")):
        _req(t.dtype == torch.bfloat16 and tuple(t.shape) == (batch, 512), f"{n}: bf16 [batch, 512]")
    _req(gate.dtype == torch.bfloat16 and gate.shape == q.shape, "gate: bf16 like q")
    _req(keys.dtype == torch.bfloat16 and keys.dim() == 2 and keys.shape[1] == 512
         and values.shape == keys.shape and values.dtype == keys.dtype, "caches: bf16 [slots, 512]")
    _req(append.dtype == torch.int64 and append.numel() == batch, "append: int64 [batch]")
    _req(table.dtype == torch.int64 and table.dim() == 2 and table.shape[0] == batch,
         "table: int64 [batch, context]")
    _req(mask.dtype == torch.float32 and mask.shape == table.shape, "mask: fp32 [batch, context]")
    context = table.shape[1]
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        n = lib().ifattn_gated_paged_attention_workspace_size(batch, context)
        workspace = torch.empty(max(int(n), 16), dtype=torch.uint8, device=q.device)
    check(lib().ifattn_gated_paged_attention_bf16(
        _ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(keys), _ptr(values), _ptr(append), _ptr(table),
        _ptr(mask), _ptr(out), batch, keys.shape[0], context, _ptr(workspace), workspace.numel(),
        _stream(stream)), "ifattn_gated_paged_attention_bf16")
    return out


def qk_norm_rope_gate(packed_q, k, q_gamma, k_gamma, positions, stream=None):
    """Qwen attention producer (inferfabric_acl_attention_qk_prepare): per-head
    RMS norm of q (packed [batch, 8, 512], query then gate channels) and k
    [batch, 2, 256], partial RoPE at ``positions`` [batch] int64, sigmoid gate.
    Returns (q [batch, 8, 256], k [batch, 2, 256], gate [batch, 8, 256]) bf16."""
    _dev(packed_q, k, q_gamma, k_gamma, positions)
    _req(packed_q.dtype == torch.bfloat16 and packed_q.dim() == 3
         and tuple(packed_q.shape[1:]) == (8, 512), "packed_q: bf16 [batch, 8, 512]")
    batch = packed_q.shape[0]
    _req(k.dtype == torch.bfloat16 and tuple(k.shape) == (batch, 2, 256), "k: bf16 [batch, 2, 256]")
    for g, n in ((q_gamma, "q_gamma"), (k_gamma, "k_gamma")):
        _req(g.dtype == torch.float32 and g.numel() == 256, f"{n}: fp32 [256]")
    _req(positions.dtype == torch.int64 and positions.numel() == batch, "positions: int64 [batch]")
    q_out = torch.empty((batch, 8, 256), dtype=torch.bfloat16, device=packed_q.device)
    k_out = torch.empty((batch, 2, 256), dtype=torch.bfloat16, device=packed_q.device)
    gate = torch.empty_like(q_out)
    check(lib().ifattn_qk_norm_rope_gate_bf16(
        _ptr(packed_q), _ptr(k), _ptr(q_gamma), _ptr(k_gamma), _ptr(positions), _ptr(q_out),
        _ptr(k_out), _ptr(gate), batch, _stream(stream)), "ifattn_qk_norm_rope_gate_bf16")
    return q_out, k_out, gate


# ---------------------------------------------------------------- varlen prefill

def prefill_workspace(num_seqs, total_q, q_heads, head_dim, max_kv_len, device="cuda"):
    n = lib().ifattn_varlen_prefill_workspace_size(num_seqs, total_q, q_heads, head_dim, max_kv_len)
    return torch.empty(max(int(n), 16), dtype=torch.uint8, device=device)


def varlen_prefill(q, k_cache, v_cache, block_tables, cu_seqlens_q, kv_lens, max_q_len,
                   max_kv_len, scale=None, out=None, workspace=None, stream=None):
    """Packed chunked prefill (+ decode rows). q [total_q, q_heads, head_dim] bf16."""
    _dev(q, k_cache, v_cache, block_tables, cu_seqlens_q, kv_lens, out, workspace)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3, "q: bf16 [total_q, q_heads, head_dim]")
    tq, hq, hd = q.shape
    _req(k_cache.dtype == torch.bfloat16 and k_cache.dim() == 4 and k_cache.shape == v_cache.shape
         and k_cache.shape[3] == hd, "caches: bf16 [num_blocks, block_size, kv_heads, head_dim]")
    nb, bs, hkv, _ = k_cache.shape
    _req(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.dim() == 1, "cu_seqlens_q: int32")
    ns = cu_seqlens_q.numel() - 1
    _check_tables(block_tables, kv_lens, ns, bs, max_kv_len)
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = prefill_workspace(ns, tq, hq, hd, max_kv_len, q.device)
    st = lib().ifattn_varlen_prefill_bf16(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables), block_tables.shape[1],
        _ptr(cu_seqlens_q), _ptr(kv_lens), _ptr(out), ns, tq, max_q_len, max_kv_len, hq, hkv, hd,
        bs, nb, float(scale), _ptr(workspace), workspace.numel(), _stream(stream))
    check(st, "ifattn_varlen_prefill_bf16")
    return out


# ---------------------------------------------------------------- MLA decode

def mla_workspace(num_seqs, heads, max_context, block_size, device="cuda"):
    n = lib().ifattn_mla_decode_workspace_size(num_seqs, heads, max_context, block_size)
    return torch.empty(max(int(n), 16), dtype=torch.uint8, device=device)


def mla_decode(q, cache, block_tables, seq_lens, max_context, scale=None, out=None,
               workspace=None, stream=None):
    """q [num_seqs, heads, 576] bf16; cache bf16 [blocks, bs, 576] or uint8 [blocks, bs, 656]."""
    c8 = cache.dtype == torch.uint8
    _dev(q, cache, block_tables, seq_lens, out, workspace)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3 and q.shape[2] == 576,
         "q: bf16 [num_seqs, heads, 576]")
    ns, h, _ = q.shape
    _req(cache.dim() == 3 and cache.shape[2] == (656 if c8 else 576)
         and cache.dtype in (torch.uint8, torch.bfloat16), "cache: bf16 [.., 576] or uint8 [.., 656]")
    nb, bs, _ = cache.shape
    _check_tables(block_tables, seq_lens, ns, bs, max_context)
    if scale is None:
        scale = 1.0 / math.sqrt(192.0)
    if out is None:
        out = torch.empty((ns, h, 512), dtype=torch.bfloat16, device=q.device)
    _req(tuple(out.shape) == (ns, h, 512) and out.dtype == torch.bfloat16, "out: bf16 [n, heads, 512]")
    if workspace is None:
        workspace = mla_workspace(ns, h, max_context, bs, q.device)
    fn = lib().ifattn_mla_decode_c8 if c8 else lib().ifattn_mla_decode_bf16
    st = fn(_ptr(q), _ptr(cache), _ptr(block_tables), block_tables.shape[1], _ptr(seq_lens),
            _ptr(out), ns, h, bs, nb, max_context, float(scale), _ptr(workspace),
            workspace.numel(), _stream(stream))
    check(st, "ifattn_mla_decode")
    return out


def mla_decode_step(q, x_new, gamma, cos, sin, cache, block_tables, seq_lens, max_context,
                    eps=1e-5, scale=None, out=None, workspace=None, stream=None):
    """Fused MLA decode step: x_new [num_seqs, 576] bf16 rows are normalized
    (gamma [512] bf16, eps), roped (cos/sin [num_seqs, 64] bf16) and stored at
    each sequence's last position seq_lens[s] - 1, then attended over with
    q [num_seqs, heads, 576]. cache bf16 [blocks, bs, 576] or uint8 [blocks, bs, 656].
    The block holding each sequence's last position must not be shared with
    another sequence of the call."""
    c8 = cache.dtype == torch.uint8
    _dev(q, x_new, gamma, cos, sin, cache, block_tables, seq_lens, out, workspace)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3 and q.shape[2] == 576,
         "q: bf16 [num_seqs, heads, 576]")
    ns, h, _ = q.shape
    _req(x_new.dtype == torch.bfloat16 and tuple(x_new.shape) == (ns, 576), "x_new: bf16 [num_seqs, 576]")
    _req(gamma.dtype == torch.bfloat16 and gamma.numel() == 512, "gamma: bf16 [512]")
    for t, n in ((cos, "cos"), (sin, "sin")):
        _req(t.dtype == torch.bfloat16 and tuple(t.shape) == (ns, 64), f"{n}: bf16 [num_seqs, 64]")
    _req(cache.dim() == 3 and cache.shape[2] == (656 if c8 else 576)
         and cache.dtype in (torch.uint8, torch.bfloat16), "cache: bf16 [.., 576] or uint8 [.., 656]")
    nb, bs, _ = cache.shape
    _check_tables(block_tables, seq_lens, ns, bs, max_context)
    if scale is None:
        scale = 1.0 / math.sqrt(192.0)
    if out is None:
        out = torch.empty((ns, h, 512), dtype=torch.bfloat16, device=q.device)
    _req(tuple(out.shape) == (ns, h, 512) and out.dtype == torch.bfloat16, "out: bf16 [n, heads, 512]")
    if workspace is None:
        workspace = mla_workspace(ns, h, max_context, bs, q.device)
    st = lib().ifattn_mla_decode_step(
        _ptr(q), _ptr(x_new), _ptr(gamma), _ptr(cos), _ptr(sin), float(eps), _ptr(cache), int(c8),
        _ptr(block_tables), block_tables.shape[1], _ptr(seq_lens), _ptr(out), ns, h, bs, nb,
        max_context, float(scale), _ptr(workspace), workspace.numel(), _stream(stream))
    check(st, "ifattn_mla_decode_step")
    return out


def mla_attention(q, cache, block_tables, kv_lens, max_context, cu_seqlens=None, indices=None,
                  window=0, sink_keys=None, sink_values=None, scale=None, out=None,
                  workspace=None, stream=None, row_scales=None, bits=8):
    """Packed-MLA attention over query rows.

    q [rows, heads, 576] bf16; rows per sequence from cu_seqlens int32 [seqs+1]
    (None: one row per sequence); kv_lens int32 [seqs]. bf16 caches
    [blocks, bs, 576] take the window path (``window`` 0 = all keys); packed C8
    caches uint8 [blocks, bs, 656] take the sparse path with ``indices`` int32
    [rows, topk]; row-quantized caches uint8 [blocks, bs, 576 * bits / 8] with
    ``row_scales`` fp32 [blocks * bs] take the window path, dequantized in
    registers. sink_keys [n, 576] / sink_values [n, 512] bf16 (n <= 128) are
    optional. Returns out [rows, heads, 512] bf16.
    """
    rowq = row_scales is not None
    c8 = cache.dtype == torch.uint8 and not rowq
    _dev(q, cache, block_tables, kv_lens, cu_seqlens, indices, sink_keys, sink_values, out, workspace,
         row_scales)
    _req(q.dtype == torch.bfloat16 and q.dim() == 3 and q.shape[2] == 576, "q: bf16 [rows, heads, 576]")
    rows, h, _ = q.shape
    if rowq:
        _req(bits in (8, 4) and cache.dtype == torch.uint8 and cache.dim() == 3
             and cache.shape[2] == 576 * bits // 8, "row-quantized cache: uint8 [.., 576 * bits / 8]")
        _req(row_scales.dtype == torch.float32 and row_scales.numel() == cache.shape[0] * cache.shape[1],
             "row_scales: fp32 [blocks * block_size]")
        _req(indices is None, "row-quantized caches take windows")
    else:
        _req(cache.dim() == 3 and cache.shape[2] == (656 if c8 else 576)
             and cache.dtype in (torch.uint8, torch.bfloat16), "cache: bf16 [.., 576] or uint8 [.., 656]")
        _req(c8 == (indices is not None), "C8 caches take index lists, bf16 caches take windows")
    nb, bs, _ = cache.shape
    seqs = rows if cu_seqlens is None else cu_seqlens.numel() - 1
    _req(cu_seqlens is None or (cu_seqlens.dtype == torch.int32 and seqs >= 1),
         "cu_seqlens: int32 [seqs + 1]")
    _check_tables(block_tables, kv_lens, seqs, bs, max_context)
    topk = 0
    if indices is not None:
        _req(indices.dtype == torch.int32 and indices.dim() == 2 and indices.shape[0] == rows,
             "indices: int32 [rows, topk]")
        topk = indices.shape[1]
    ns = 0
    if sink_keys is not None:
        ns = sink_keys.shape[0]
        _req(sink_keys.dtype == torch.bfloat16 and tuple(sink_keys.shape) == (ns, 576)
             and sink_values is not None and sink_values.dtype == torch.bfloat16
             and tuple(sink_values.shape) == (ns, 512), "sinks: bf16 keys [n, 576], values [n, 512]")
    if scale is None:
        scale = 1.0 / math.sqrt(192.0)
    if out is None:
        out = torch.empty((rows, h, 512), dtype=torch.bfloat16, device=q.device)
    _req(tuple(out.shape) == (rows, h, 512) and out.dtype == torch.bfloat16, "out: bf16 [rows, heads, 512]")
    if workspace is None:
        n = lib().ifattn_mla_attention_workspace_size(rows, h, max_context, int(window), topk, ns, bs)
        workspace = torch.empty(max(int(n), 16), dtype=torch.uint8, device=q.device)
    if rowq:
        st = lib().ifattn_mla_window_attention_rowq(
            _ptr(q), _ptr(cache), _ptr(row_scales), int(bits), _ptr(block_tables),
            block_tables.shape[1], _ptr(cu_seqlens), _ptr(kv_lens), seqs, rows, int(window),
            _ptr(sink_keys), _ptr(sink_values), ns, _ptr(out), h, bs, nb, max_context, float(scale),
            _ptr(workspace), workspace.numel(), _stream(stream))
    elif c8:
        st = lib().ifattn_mla_sparse_attention_c8(
            _ptr(q), _ptr(cache), _ptr(indices), topk, _ptr(block_tables), block_tables.shape[1],
            _ptr(cu_seqlens), _ptr(kv_lens), seqs, rows, _ptr(sink_keys), _ptr(sink_values), ns,
            _ptr(out), h, bs, nb, max_context, float(scale), _ptr(workspace), workspace.numel(),
            _stream(stream))
    else:
        st = lib().ifattn_mla_window_attention_bf16(
            _ptr(q), _ptr(cache), _ptr(block_tables), block_tables.shape[1], _ptr(cu_seqlens),
            _ptr(kv_lens), seqs, rows, int(window), _ptr(sink_keys), _ptr(sink_values), ns,
            _ptr(out), h, bs, nb, max_context, float(scale), _ptr(workspace), workspace.numel(),
            _stream(stream))
    check(st, "ifattn_mla_attention")
    return out


# ---------------------------------------------------------------- slot reuse

def page_reset(field, spans, stream=None, status=None):
    """Zero the {offset, bytes} spans (uint64 [count, 2] on the device, e.g. from
    host.page_spans) of a device state tensor, viewed as bytes. With ``status``
    (int32 [1] on the device) the plan is validated first and an invalid plan
    zeroes nothing (status = 1 + first bad span)."""
    _dev(field, spans, status)
    _req(spans.dtype in (torch.int64, torch.uint64) and spans.dim() == 2 and spans.shape[1] == 2,
         "spans: uint64/int64 [count, 2]")
    nbytes = field.numel() * field.element_size()
    if status is None:
        st = lib().ifattn_page_reset(_ptr(field), nbytes, _ptr(spans), spans.shape[0], _stream(stream))
    else:
        _req(status.dtype == torch.int32 and status.numel() == 1, "status: int32 [1]")
        st = lib().ifattn_page_reset_checked(_ptr(field), nbytes, _ptr(spans), spans.shape[0],
                                             _ptr(status), _stream(stream))
    check(st, "ifattn_page_reset")


def state_copy(field, ranges, stream=None, status=None):
    """Copy the {source, destination, bytes} ranges (uint64 [count, 3] on the
    device, e.g. from ResidentPages.copy_plan) inside one device state tensor.
    With ``status`` (int32 [1] on the device) the plan is validated first and an
    invalid plan copies nothing (status = 1 + first bad range)."""
    _dev(field, ranges, status)
    _req(ranges.dtype in (torch.int64, torch.uint64) and ranges.dim() == 2 and ranges.shape[1] == 3,
         "ranges: uint64/int64 [count, 3]")
    nbytes = field.numel() * field.element_size()
    if status is None:
        st = lib().ifattn_state_copy(_ptr(field), nbytes, _ptr(ranges), ranges.shape[0], _stream(stream))
    else:
        _req(status.dtype == torch.int32 and status.numel() == 1, "status: int32 [1]")
        st = lib().ifattn_state_copy_checked(_ptr(field), nbytes, _ptr(ranges), ranges.shape[0],
                                             _ptr(status), _stream(stream))
    check(st, "ifattn_state_copy")


# ---------------------------------------------------------------- legacy launchers

def cache_quantize(row, packed, scales, position, bits=8, stream=None):
    """if_cache_quantize: row bf16 [width]; packed uint8 [capacity * width*bits/8];
    scales fp32 [capacity]; position int64 [1] on the device."""
    _dev(row, packed, scales, position)
    width = row.numel()
    capacity = scales.numel()
    _req(packed.numel() >= capacity * width * bits // 8, "packed storage too small")
    lib().if_cache_quantize(_ptr(row), _ptr(packed), _ptr(scales), _ptr(position), width,
                            capacity, bits, _stream(stream))


def cache_dequantize(packed, scales, output, position, width, bits=8, stream=None):
    _dev(packed, scales, output, position)
    capacity = scales.numel()
    _req(output.numel() >= capacity * width, "output too small")
    lib().if_cache_dequantize(_ptr(packed), _ptr(scales), _ptr(output), _ptr(position), width,
                              capacity, bits, _stream(stream))


def packed_attention_metadata(positions, indices, lengths, capacity, stream=None):
    _dev(positions, indices, lengths)
    rows = positions.numel()
    _req(indices.numel() >= rows * capacity and lengths.numel() >= rows, "outputs too small")
    lib().if_packed_attention_metadata_batch(_ptr(positions), _ptr(indices), _ptr(lengths),
                                             capacity, rows, _stream(stream))
