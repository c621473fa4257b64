"""CPU oracle — TEST INFRASTRUCTURE ONLY.

ctypes binding of ``liboracle.so`` (a C++ restatement of the reference's CPU
algorithms, see oracle.cpp for the per-function citations) and of
``_ref/libref_meta.so`` (the reference's own host metadata headers compiled in
place, present only where /root/reference was available at build time).
Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg use
this package, as the checker; the product never imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_lib = None
_ref = None
_loader = None

i32, i64, u32, u64, f32, vp = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_float, C.c_void_p


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            build()
        l = C.CDLL(str(path))
        l.oracle_kv_write.argtypes = [vp, vp, vp, i64, i64, i64]
        l.oracle_quant_rows.argtypes = [vp, i64, i32, vp, vp, f32]
        l.oracle_quant_legacy.argtypes = [vp, i32, i32, vp, vp]
        l.oracle_dequant_legacy.argtypes = [vp, vp, vp, i64, i32, i32, i32]
        l.oracle_mla_pack_c8.argtypes = [vp, i64, vp]
        l.oracle_mla_norm_rope_write.argtypes = [vp, vp, vp, vp, vp, i64, f32, vp, i32, i64]
        l.oracle_paged_decode.argtypes = [vp, vp, vp, vp, vp, i32, vp, i32, vp, vp, i32, i32, i32,
                                          i32, i32, f32, i32, i32]
        l.oracle_varlen_prefill.argtypes = [vp, vp, vp, vp, i32, vp, vp, vp, i32, i32, i32, i32,
                                            i32, f32, i32]
        l.oracle_mla_decode.argtypes = [vp, vp, i32, vp, i32, vp, vp, i32, i32, i32, f32, i32]
        l.oracle_mla_attention.argtypes = [vp, vp, i32, vp, i32, vp, vp, i32, i32, vp, i32, i32,
                                           vp, vp, i32, vp, i32, i32, f32, i32]
        l.oracle_gated_attention.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32,
                                             f32, i32]
        l.oracle_qk_norm_rope_gate.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i32]
        l.oracle_hardware_threads.restype = i32
        for f in ("oracle_kv_write", "oracle_quant_rows", "oracle_quant_legacy",
                  "oracle_dequant_legacy", "oracle_mla_pack_c8", "oracle_mla_norm_rope_write",
                  "oracle_paged_decode", "oracle_gated_attention", "oracle_qk_norm_rope_gate",
                  "oracle_varlen_prefill", "oracle_mla_decode", "oracle_mla_attention"):
            getattr(l, f).restype = None
        _lib = l
    return _lib


def ref():
    """The reference's host metadata compiled in place, or None where absent."""
    global _ref
    if _ref is None:
        path = HERE / "_ref" / "libref_meta.so"
        if not path.exists():
            return None
        _ref = C.CDLL(str(path))
    return _ref


def ref_loader():
    """The reference's plug-in loader (native/src/compiled_kernel.cpp) compiled in
    place behind a C shim, or None where absent."""
    global _loader
    if _loader is None:
        path = HERE / "_ref" / "libref_loader.so"
        if not path.exists():
            return None
        l = C.CDLL(str(path))
        l.ref_loader_error.restype = C.c_char_p
        l.ref_loader_open.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p, C.POINTER(vp)]
        l.ref_loader_close.argtypes = [vp]
        l.ref_loader_prepare.argtypes = [vp, vp, u32, vp, u32, C.POINTER(vp), C.POINTER(u64)]
        l.ref_loader_enqueue.argtypes = [vp, vp, u64, vp]
        l.ref_loader_release.argtypes = [vp]
        _loader = l
    return _loader


def _p(a):
    return None if a is None else a.ctypes.data_as(vp)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def hardware_threads() -> int:
    return int(lib().oracle_hardware_threads())


def kv_write(rows, cache, slots):
    """In place: cache[slots[r]] = rows[r] (rows/cache any dtype, same row width)."""
    rows = np.ascontiguousarray(rows)
    slots = _c(slots, np.int64)
    n = rows.shape[0]
    row_bytes = rows[0].nbytes if n else 0
    num_slots = cache.nbytes // row_bytes if row_bytes else 0
    assert cache.flags.c_contiguous
    lib().oracle_kv_write(_p(rows), _p(cache), _p(slots), n, row_bytes, num_slots)


def quant_rows(x_bits, width, zero_scale=1.0):
    """Groups of `width` bf16 values -> (int8 codes, fp32 scales), round half even."""
    x = _c(x_bits, np.uint16).reshape(-1)
    groups = x.size // width
    codes = np.empty(groups * width, np.int8)
    scales = np.empty(groups, np.float32)
    lib().oracle_quant_rows(_p(x), groups, width, _p(codes), _p(scales), zero_scale)
    return codes.reshape(groups, width), scales


def quant_legacy(x_bits, bits=8):
    x = _c(x_bits, np.uint16).reshape(-1)
    packed = np.zeros(x.size * bits // 8, np.uint8)
    scale = np.zeros(1, np.float32)
    lib().oracle_quant_legacy(_p(x), x.size, bits, _p(packed), _p(scale))
    return packed, float(scale[0])


def dequant_legacy(packed, scales, last, width, bits=8):
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.float32)
    capacity = scales.size
    out = np.zeros(capacity * width, np.uint16)
    lib().oracle_dequant_legacy(_p(packed), _p(scales), _p(out), last, width, capacity, bits)
    return out


def mla_pack_c8(rows_bits):
    rows = _c(rows_bits, np.uint16).reshape(-1, 576)
    out = np.zeros((rows.shape[0], 656), np.uint8)
    lib().oracle_mla_pack_c8(_p(rows), rows.shape[0], _p(out))
    return out


def mla_norm_rope_write(x, gamma, cos, sin, slots, cache, packed, eps=1e-5):
    """In place on ``cache`` (uint8 [slots, 656] if packed else uint16 [slots, 576]):
    RMSNorm * gamma + half rotary + cache row for every row of x [rows, 576]."""
    x = _c(x, np.uint16).reshape(-1, 576)
    gamma = _c(gamma, np.uint16)
    cos = _c(cos, np.uint16).reshape(-1, 64)
    sin = _c(sin, np.uint16).reshape(-1, 64)
    slots = _c(slots, np.int64)
    assert cache.flags.c_contiguous
    num_slots = cache.shape[0]
    lib().oracle_mla_norm_rope_write(_p(x), _p(gamma), _p(cos), _p(sin), _p(slots), x.shape[0],
                                     float(eps), _p(cache), int(bool(packed)), num_slots)
    return cache


def paged_decode(q, k_cache, v_cache, block_tables, seq_lens, q_heads, kv_heads, head_dim,
                 block_size, scale, k_scale=None, v_scale=None, ref_rounding=False, threads=0):
    """fp32 output [n, q_heads, head_dim]; caches are uint16 (bf16 bits) or int8."""
    c8 = k_scale is not None
    q = _c(q, np.uint16)
    k_cache = _c(k_cache, np.int8 if c8 else np.uint16)
    v_cache = _c(v_cache, np.int8 if c8 else np.uint16)
    ks = _c(k_scale, np.float32) if c8 else None
    vs = _c(v_scale, np.float32) if c8 else None
    tables = _c(block_tables, np.int32)
    lens = _c(seq_lens, np.int32)
    n = lens.size
    out = np.zeros((n, q_heads, head_dim), np.float32)
    lib().oracle_paged_decode(_p(q), _p(k_cache), _p(v_cache), _p(ks), _p(vs), int(c8), _p(tables),
                              tables.shape[1], _p(lens), _p(out), n, q_heads, kv_heads, head_dim,
                              block_size, scale, int(ref_rounding), threads)
    return out


def varlen_prefill(q, k_cache, v_cache, block_tables, cu_seqlens, kv_lens, q_heads, kv_heads,
                   head_dim, block_size, scale, threads=0):
    q = _c(q, np.uint16)
    k_cache = _c(k_cache, np.uint16)
    v_cache = _c(v_cache, np.uint16)
    tables = _c(block_tables, np.int32)
    cu = _c(cu_seqlens, np.int32)
    kv = _c(kv_lens, np.int32)
    out = np.zeros((int(cu[-1]), q_heads, head_dim), np.float32)
    lib().oracle_varlen_prefill(_p(q), _p(k_cache), _p(v_cache), _p(tables), tables.shape[1],
                                _p(cu), _p(kv), _p(out), cu.size - 1, q_heads, kv_heads, head_dim,
                                block_size, scale, threads)
    return out


def mla_decode(q, cache, block_tables, seq_lens, heads, block_size, scale, c8=False, threads=0):
    q = _c(q, np.uint16)
    cache = _c(cache, np.uint8 if c8 else np.uint16)
    tables = _c(block_tables, np.int32)
    lens = _c(seq_lens, np.int32)
    n = lens.size
    out = np.zeros((n, heads, 512), np.float32)
    lib().oracle_mla_decode(_p(q), _p(cache), int(c8), _p(tables), tables.shape[1], _p(lens),
                            _p(out), n, heads, block_size, scale, threads)
    return out


def mla_attention(q, cache, block_tables, kv_lens, heads, block_size, scale, c8=False,
                  cu_seqlens=None, indices=None, window=0, sink_k=None, sink_v=None, threads=0):
    """fp32 [rows, heads, 512]. q [rows, heads, 576] bf16 bits; rows per sequence from
    cu_seqlens (None: one row per sequence); indices [rows, topk] for sparse rows."""
    q = _c(q, np.uint16).reshape(-1, heads, 576)
    rows = q.shape[0]
    cache = _c(cache, np.uint8 if c8 else np.uint16)
    tables = _c(block_tables, np.int32)
    kv = _c(kv_lens, np.int32)
    cu = None if cu_seqlens is None else _c(cu_seqlens, np.int32)
    idx = None if indices is None else _c(indices, np.int32).reshape(rows, -1)
    topk = 0 if idx is None else idx.shape[1]
    sk = None if sink_k is None else _c(sink_k, np.uint16).reshape(-1, 576)
    sv = None if sink_v is None else _c(sink_v, np.uint16).reshape(-1, 512)
    ns = 0 if sk is None else sk.shape[0]
    out = np.zeros((rows, heads, 512), np.float32)
    lib().oracle_mla_attention(_p(q), _p(cache), int(c8), _p(tables), tables.shape[1], _p(cu),
                               _p(kv), kv.size, rows, _p(idx), topk, int(window), _p(sk), _p(sv),
                               ns, _p(out), heads, block_size, float(scale), threads)
    return out


def gated_attention(q, keys, values, table, mask, gate, hq=8, hkv=2, d=256, scale=0.0625,
                    threads=0):
    """fp32 [batch, hq, d]: softmax(q.K[table]*scale + mask) V[table], times gate.
    q/gate bf16 bits [batch, hq, d]; keys/values bf16 bits [slots, hkv*d];
    table int64, mask fp32 [batch, context]."""
    q = _c(q, np.uint16)
    keys = _c(keys, np.uint16)
    values = _c(values, np.uint16)
    table = _c(table, np.int64)
    mask = _c(mask, np.float32)
    gate = _c(gate, np.uint16)
    batch, context = table.shape
    out = np.zeros((batch, hq, d), np.float32)
    lib().oracle_gated_attention(_p(q), _p(keys), _p(values), _p(table), _p(mask), _p(gate),
                                 _p(out), batch, context, hq, hkv, d, float(scale), threads)
    return out


def qk_norm_rope_gate(packed_q, k, q_gamma, k_gamma, positions):
    """(q [batch, 8, 256], k [batch, 2, 256], gate [batch, 8, 256]) as bf16 bits from
    packed q bf16 bits [batch, 8, 512], k bf16 bits [batch, 2, 256], fp32 gammas [256]
    and int64 positions [batch]."""
    packed_q = _c(packed_q, np.uint16)
    k = _c(k, np.uint16)
    q_gamma = _c(q_gamma, np.float32)
    k_gamma = _c(k_gamma, np.float32)
    positions = _c(positions, np.int64)
    batch = positions.shape[0]
    q_out = np.zeros((batch, 8, 256), np.uint16)
    k_out = np.zeros((batch, 2, 256), np.uint16)
    gate = np.zeros((batch, 8, 256), np.uint16)
    lib().oracle_qk_norm_rope_gate(_p(packed_q), _p(k), _p(q_gamma), _p(k_gamma), _p(positions),
                                   _p(q_out), _p(k_out), _p(gate), batch)
    return q_out, k_out, gate
