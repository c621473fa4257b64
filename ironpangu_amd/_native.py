"""ctypes binding of ``libifattn_hip.so`` (the C ABI in include/ifattn.h,
include/ifattn_host.h and include/cache_quantization.h).

The library must be built in-tree (``python -m ironpangu_amd.build`` or
``__graft_entry__.build()``); there is no fallback implementation, and
``lib()`` raises if it is missing. ``torch`` is imported first when available
so that the library binds to the HIP runtime torch already loaded (both carry
the soname ``libamdhip64.so.7``).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import os

PKG = Path(__file__).resolve().parent
# IFATTN_LIBRARY may point at another build of the same C ABI (e.g. a tuning build).
LIB_PATH = Path(os.environ.get("IFATTN_LIBRARY", str(PKG / "libifattn_hip.so")))

_lib = None

i32, i64, u32, u64, f32, vp = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_float, C.c_void_p
pi32, pi64, pu32, pu64 = C.POINTER(i32), C.POINTER(i64), C.POINTER(u32), C.POINTER(u64)


class SequenceSlice(C.Structure):
    _fields_ = [("resident", u32), ("position", u32), ("tokens", u32), ("sample", i32)]


class StateGeometry(C.Structure):
    _fields_ = [("format", u32), ("page_tokens", u32), ("row_bytes", u32), ("num_blocks", u32),
                ("table_entries", u32), ("heads", u32), ("cache_bytes", u64)]


class StateBuffers(C.Structure):
    _fields_ = [(n, vp) for n in ("cache", "table", "scales", "query", "out", "indices", "kv_len",
                                  "sink_keys", "sink_values")]


# name -> (restype, argtypes)
SIGNATURES = {
    "ifattn_abi_version": (i32, []),
    "ifattn_last_error": (C.c_char_p, []),
    "ifattn_kv_cache_write": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, i64, vp]),
    "ifattn_kv_cache_write_c8": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i64, i32, i32, i64, vp]),
    "ifattn_mla_cache_write_c8": (i32, [vp, vp, vp, i32, i64, i64, vp]),
    "ifattn_mla_norm_rope_cache_write": (i32, [vp, vp, vp, vp, vp, i32, i64, f32, vp, i32, i64, vp]),
    "ifattn_paged_decode_workspace_size": (u64, [i32, i32, i32, i32]),
    "ifattn_paged_decode_bf16": (i32, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i64,
                                       i32, f32, vp, u64, vp]),
    "ifattn_paged_decode_step_bf16": (i32, [vp, vp, vp, vp, vp, vp, i32, i64, vp, i32, vp, vp, i32,
                                            i32, i32, i32, i32, i64, i32, f32, vp, u64, vp]),
    "ifattn_paged_decode_step_bf16_noalloc": (i32, [vp, vp, vp, vp, vp, vp, i32, i64, vp, i32, vp, vp,
                                                    i32, i32, i32, i32, i32, i64, i32, f32, vp]),
    "ifattn_paged_decode_c8": (i32, [vp, vp, vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32,
                                     i64, i32, f32, vp, u64, vp]),
    "ifattn_gated_paged_attention_workspace_size": (u64, [i64, i64]),
    "ifattn_gated_paged_attention_bf16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64,
                                                i64, vp, u64, vp]),
    "ifattn_qk_norm_rope_gate_bf16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i64, vp]),
    "ifattn_varlen_prefill_workspace_size": (u64, [i32, i32, i32, i32, i32]),
    "ifattn_varlen_prefill_bf16": (i32, [vp, vp, vp, vp, i32, vp, vp, vp, i32, i32, i32, i32, i32,
                                         i32, i32, i32, i64, f32, vp, u64, vp]),
    "ifattn_mla_decode_workspace_size": (u64, [i32, i32, i32, i32]),
    "ifattn_mla_decode_bf16": (i32, [vp, vp, vp, i32, vp, vp, i32, i32, i32, i64, i32, f32, vp,
                                     u64, vp]),
    "ifattn_mla_decode_c8": (i32, [vp, vp, vp, i32, vp, vp, i32, i32, i32, i64, i32, f32, vp, u64,
                                   vp]),
    "ifattn_mla_decode_step": (i32, [vp, vp, vp, vp, vp, f32, vp, i32, vp, i32, vp, vp, i32, i32, i32,
                                     i64, i32, f32, vp, u64, vp]),
    "ifattn_mla_attention_workspace_size": (u64, [i32, i32, i32, i32, i32, i32, i32]),
    "ifattn_mla_window_attention_bf16": (i32, [vp, vp, vp, i32, vp, vp, i32, i32, i32, vp, vp, i32,
                                               vp, i32, i32, i64, i32, f32, vp, u64, vp]),
    "ifattn_mla_window_attention_rowq": (i32, [vp, vp, vp, i32, vp, i32, vp, vp, i32, i32, i32, vp,
                                               vp, i32, vp, i32, i32, i64, i32, f32, vp, u64, vp]),
    "ifattn_mla_sparse_attention_c8": (i32, [vp, vp, vp, i32, vp, i32, vp, vp, i32, i32, vp, vp,
                                             i32, vp, i32, i32, i64, i32, f32, vp, u64, vp]),
    "ifattn_page_reset": (i32, [vp, u64, vp, u64, vp]),
    "ifattn_state_copy": (i32, [vp, u64, vp, u64, vp]),
    "ifattn_page_reset_checked": (i32, [vp, u64, vp, u64, vp, vp]),
    "ifattn_state_copy_checked": (i32, [vp, u64, vp, u64, vp, vp]),
    "if_cache_quantize": (None, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "if_cache_dequantize": (None, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "if_packed_attention_metadata": (None, [vp, vp, vp, u32, vp]),
    "if_packed_attention_metadata_batch": (None, [vp, vp, vp, u32, u32, vp]),
    "ifattn_pages_create": (i32, [u32, u32, u32, i32, C.POINTER(vp)]),
    "ifattn_pages_destroy": (None, [vp]),
    "ifattn_pages_select": (i32, [vp, u32]),
    "ifattn_pages_bind": (i32, [vp, pi32, u64]),
    "ifattn_pages_release": (i32, [vp, u32]),
    "ifattn_pages_selected": (i32, [vp, pu32]),
    "ifattn_attention_state_create": (i32, [u32, u32, i32, u32, i32, u32, u32, C.POINTER(vp)]),
    "ifattn_attention_state_destroy": (None, [vp]),
    "ifattn_attention_state_geometry_of": (i32, [vp, C.POINTER(StateGeometry)]),
    "ifattn_attention_state_pages": (i32, [vp, C.POINTER(vp)]),
    "ifattn_attention_state_append": (i32, [vp, u32, pu64]),
    "ifattn_attention_state_blocks": (i32, [vp, pi32, u32, pu32]),
    "ifattn_attention_state_buffers_of": (i32, [vp, C.POINTER(StateBuffers)]),
    "ifattn_attention_state_upload_table": (i32, [vp, vp]),
    "ifattn_attention_state_set_length": (i32, [vp, i32, vp]),
    "ifattn_attention_state_attend": (i32, [vp, i32, i32, vp]),
    "ifattn_pages_owned": (i32, [vp, u32, pi32, u64, pu64]),
    "ifattn_pages_append": (i32, [vp, u32, u32, pu64]),
    "ifattn_pages_slot_mapping": (i32, [vp, pi32, pi32, u64, pi64]),
    "ifattn_pages_batch_table": (i32, [vp, pi32, u64, u32, i32, pi32]),
    "ifattn_pages_copy_plan": (i32, [vp, u32, u32, u32, i32, u64, pu64, u64, pu64]),
    "ifattn_page_spans": (i32, [pi32, u64, u64, u64, pu64, u64, pu64]),
    "ifattn_window_layout": (i32, [u32, u32, u32, u32, pu32, pu32]),
    "ifattn_window_table": (i32, [u32, u32, u32, u32, pi32, u64, pi32]),
    "ifattn_window_slots": (i32, [u32, u32, u32, u32, pi32, u64, pu32, u64, pi64]),
    "ifattn_sequence_batch_make": (i32, [C.POINTER(SequenceSlice), u64, u32, u32, u32, u64, pi32,
                                         pi32, pi32, pi32, pi32, pi32, pi32, pi64, pu32, pu32,
                                         pu64, pu64]),
}


class IfattnError(RuntimeError):
    def __init__(self, status: int, where: str):
        msg = lib().ifattn_last_error().decode(errors="replace")
        super().__init__(f"{where} failed with status {status}: {msg}")
        self.status = status


def lib():
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m ironpangu_amd.build` "
                "(there is no non-native fallback)")
        try:
            import torch  # noqa: F401  (share torch's HIP runtime)
        except ImportError:
            pass
        l = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            if not hasattr(l, name):
                continue  # absent entry points raise AttributeError when called
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(status: int, where: str) -> None:
    if status != 0:
        raise IfattnError(status, where)
