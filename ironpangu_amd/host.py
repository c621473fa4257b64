"""Host metadata mirror of the reference's page-binding and packed-batch
classes, backed by the native implementation in ``libifattn_hip.so``
(include/ifattn_host.h). Names, argument meaning and error behaviour follow
native/src/page_binding.h (ResidentPages, page_spans, copy_plan) and
native/include/sequence_batch.h (SequenceBatch::make): invalid input raises
``MetadataError`` (the reference throws std::runtime_error) and leaves the
previous state untouched.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._native import SequenceSlice, StateBuffers, StateGeometry, lib


class MetadataError(RuntimeError):
    pass


def _check(status: int) -> None:
    if status != 0:
        raise MetadataError(lib().ifattn_last_error().decode(errors="replace"))


def _i32(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(C.POINTER(C.c_int32))


class ResidentPages:
    """Per-resident page ownership (native/src/page_binding.h:65-188).

    ``shared=False``: resident r owns a fixed partition of the pool and may
    permute pages inside it. ``shared=True``: residents claim unowned pages.
    """

    def __init__(self, page_tokens: int, logical_tokens: int, slots: int, shared: bool = False):
        self._h = C.c_void_p()
        self.page_tokens = page_tokens
        self.logical_tokens = logical_tokens
        self.slots = slots
        _check(lib().ifattn_pages_create(page_tokens, logical_tokens, slots, int(shared),
                                         C.byref(self._h)))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().ifattn_pages_destroy(h)
            self._h = None

    def select(self, slot: int) -> None:
        _check(lib().ifattn_pages_select(self._h, slot))

    def bind(self, pages) -> None:
        a, p = _i32(pages)
        _check(lib().ifattn_pages_bind(self._h, p, a.size))

    def release(self, slot: int) -> None:
        _check(lib().ifattn_pages_release(self._h, slot))

    def pages(self, slot: int) -> list:
        n = C.c_uint64()
        _check(lib().ifattn_pages_owned(self._h, slot, None, 0, C.byref(n)))
        a = np.zeros(max(n.value, 1), np.int32)
        _check(lib().ifattn_pages_owned(self._h, slot, a.ctypes.data_as(C.POINTER(C.c_int32)),
                                        a.size, C.byref(n)))
        return a[: n.value].tolist()

    def append(self, *args) -> int:
        """append(position) for the selected resident or append(slot, position)."""
        slot, pos = (0xFFFFFFFF, args[0]) if len(args) == 1 else args
        if pos < 0 or slot < 0:
            raise MetadataError("negative slot or position")
        out = C.c_uint64()
        _check(lib().ifattn_pages_append(self._h, slot, pos, C.byref(out)))
        return out.value

    def slot_mapping(self, row_residents, positions) -> np.ndarray:
        r, rp = _i32(row_residents)
        q, qp = _i32(positions)
        if r.size != q.size:
            raise MetadataError("row residents and positions differ in length")
        out = np.zeros(r.size, np.int64)
        _check(lib().ifattn_pages_slot_mapping(self._h, rp, qp, r.size,
                                               out.ctypes.data_as(C.POINTER(C.c_int64))))
        return out

    def batch_table(self, residents, entries: int, ring: bool = False) -> np.ndarray:
        r, rp = _i32(residents)
        out = np.zeros(r.size * entries, np.int32)
        _check(lib().ifattn_pages_batch_table(self._h, rp, r.size, entries, int(ring),
                                              out.ctypes.data_as(C.POINTER(C.c_int32))))
        return out

    def copy_plan(self, source: int, destination: int, completed_tokens: int, windowed: bool,
                  field_bytes: int) -> list:
        n = C.c_uint64()
        _check(lib().ifattn_pages_copy_plan(self._h, source, destination, completed_tokens,
                                            int(windowed), field_bytes, None, 0, C.byref(n)))
        buf = np.zeros(max(3 * n.value, 3), np.uint64)
        _check(lib().ifattn_pages_copy_plan(self._h, source, destination, completed_tokens,
                                            int(windowed), field_bytes,
                                            buf.ctypes.data_as(C.POINTER(C.c_uint64)), n.value,
                                            C.byref(n)))
        return [tuple(int(x) for x in buf[3 * i:3 * i + 3]) for i in range(n.value)]


def page_spans(pages, page_bytes: int, field_bytes: int) -> list:
    """Sorted, coalesced byte spans of owned pages (native/src/page_binding.h:19-35)."""
    a, p = _i32(pages)
    n = C.c_uint64()
    _check(lib().ifattn_page_spans(p, a.size, page_bytes, field_bytes, None, 0, C.byref(n)))
    buf = np.zeros(max(2 * n.value, 2), np.uint64)
    _check(lib().ifattn_page_spans(p, a.size, page_bytes, field_bytes,
                                   buf.ctypes.data_as(C.POINTER(C.c_uint64)), n.value, C.byref(n)))
    return [(int(buf[2 * i]), int(buf[2 * i + 1])) for i in range(n.value)]


class WindowLayout:
    """Page ring of a sliding-window cache
    (native/include/sliding_window_layout.h:9-33): ``physical_pages`` pages
    hold the window plus a chunk of rows written before they are queried; the
    block table keeps absolute logical pages, logical page l -> ring page
    l % physical_pages. ``owned`` optionally names the resident's page ids
    (one per ring page), as a ResidentPages ring table does."""

    def __init__(self, context: int, window: int, chunk: int, page_tokens: int):
        pages, entries = C.c_uint32(), C.c_uint32()
        _check(lib().ifattn_window_layout(context, window, chunk, page_tokens, C.byref(pages),
                                          C.byref(entries)))
        self.context, self.window, self.chunk, self.page_tokens = context, window, chunk, page_tokens
        self.physical_pages, self.table_entries = pages.value, entries.value

    def _owned(self, owned):
        if owned is None:
            return None, None, 0
        a, p = _i32(owned)
        return a, p, a.size

    def table(self, owned=None) -> np.ndarray:
        keep, p, n = self._owned(owned)
        out = np.zeros(self.table_entries, np.int32)
        _check(lib().ifattn_window_table(self.context, self.window, self.chunk, self.page_tokens,
                                         p, n, out.ctypes.data_as(C.POINTER(C.c_int32))))
        return out

    def slots(self, positions, owned=None) -> np.ndarray:
        keep, p, n = self._owned(owned)
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        out = np.zeros(pos.size, np.int64)
        _check(lib().ifattn_window_slots(self.context, self.window, self.chunk, self.page_tokens,
                                         p, n, pos.ctypes.data_as(C.POINTER(C.c_uint32)), pos.size,
                                         out.ctypes.data_as(C.POINTER(C.c_int64))))
        return out

    def physical_page(self, logical: int) -> int:
        if logical < 0 or logical >= self.table_entries:
            raise MetadataError("sliding page bounds")
        return logical % self.physical_pages

    def append(self, position: int) -> int:
        return int(self.slots([position])[0]) if 0 <= position < self.context else \
            _raise("sliding append bounds")


def _raise(msg):
    raise MetadataError(msg)


@dataclass
class SequenceBatch:
    """Packed varlen layout (native/include/sequence_batch.h:15-59); ``starts``
    is cu_seqlens_q."""
    starts: list = field(default_factory=list)
    residents: list = field(default_factory=list)
    positions: list = field(default_factory=list)
    row_residents: list = field(default_factory=list)
    query_ends: list = field(default_factory=list)
    prior_lengths: list = field(default_factory=list)
    kv_lengths: list = field(default_factory=list)
    lengths: list = field(default_factory=list)
    sample_rows: list = field(default_factory=list)
    sample_residents: list = field(default_factory=list)

    @staticmethod
    def make(sequences, resident_capacity: int, token_budget: int, context: int) -> "SequenceBatch":
        """sequences: iterable of (resident, position, tokens, sample)."""
        seqs = list(sequences)
        n = len(seqs)
        arr = (SequenceSlice * max(n, 1))()
        for i, (r, p, t, s) in enumerate(seqs):
            if min(r, p, t) < 0 or max(r, p, t) > 0xFFFFFFFF:
                raise MetadataError("sequence fields must be uint32")
            arr[i] = SequenceSlice(r, p, t, int(bool(s)))
        total = sum(int(s[2]) for s in seqs) if seqs else 0
        cap = max(total, 1) if total < (1 << 31) else 1

        def buf(k, dt):
            return np.zeros(max(k, 1), dt)

        starts, qe, pr, kv, res = (buf(n + 1, np.int32), buf(n, np.int32), buf(n, np.int32),
                                   buf(n, np.int32), buf(n, np.int32))
        pos, rr, lens = buf(cap, np.int32), buf(cap, np.int32), buf(cap, np.int64)
        sr, sres = buf(n, np.uint32), buf(n, np.uint32)
        rows, samples = C.c_uint64(), C.c_uint64()

        def p(a, ct):
            return a.ctypes.data_as(C.POINTER(ct))

        _check(lib().ifattn_sequence_batch_make(
            arr if n else None, n, resident_capacity, token_budget, context, cap,
            p(starts, C.c_int32), p(qe, C.c_int32), p(pr, C.c_int32), p(kv, C.c_int32),
            p(res, C.c_int32), p(pos, C.c_int32), p(rr, C.c_int32), p(lens, C.c_int64),
            p(sr, C.c_uint32), p(sres, C.c_uint32), C.byref(rows), C.byref(samples)))
        r, s = rows.value, samples.value
        return SequenceBatch(starts[: n + 1].tolist(), res[:n].tolist(), pos[:r].tolist(),
                             rr[:r].tolist(), qe[:n].tolist(), pr[:n].tolist(), kv[:n].tolist(),
                             lens[:r].tolist(), sr[:s].tolist(), sres[:s].tolist())


class _BorrowedPages(ResidentPages):
    """ResidentPages view of a page binding owned by an AttentionState."""

    def __init__(self, handle, page_tokens, logical_tokens, slots, owner):
        self._h = handle
        self.page_tokens, self.logical_tokens, self.slots = page_tokens, logical_tokens, slots
        self._owner = owner  # keeps the state (and the binding) alive

    def __del__(self):
        pass


class AttentionState:
    """One MLA attention layer's state (native/src/openpangu_decoder_state.h:16-48):
    cache, page binding, block table, query/output/index/length buffers and 128
    sink rows, over include/ifattn_state.h. Device buffers are allocated on the
    current device at the first call that needs them."""

    FORMATS = {0: "bf16", 1: "packed_c8", 2: "row_quant"}

    def __init__(self, bits=16, capacity=512, packed=False, residents=1, shared=False, context=0,
                 heads=6):
        self._h = C.c_void_p()
        _check(lib().ifattn_attention_state_create(bits, capacity, int(packed), residents,
                                                   int(shared), context, heads, C.byref(self._h)))
        g = StateGeometry()
        _check(lib().ifattn_attention_state_geometry_of(self._h, C.byref(g)))
        self.geometry = {f: getattr(g, f) for f, _ in StateGeometry._fields_}
        self.format = self.FORMATS[g.format]
        self.capacity, self.context, self.residents = capacity, context, residents
        ph = C.c_void_p()
        _check(lib().ifattn_attention_state_pages(self._h, C.byref(ph)))
        self.page_binding = _BorrowedPages(ph, g.page_tokens, capacity, residents, self)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().ifattn_attention_state_destroy(h)
            self._h = None

    def append(self, position: int) -> int:
        out = C.c_uint64()
        _check(lib().ifattn_attention_state_append(self._h, position, C.byref(out)))
        return out.value

    def blocks(self) -> np.ndarray:
        n = C.c_uint32()
        _check(lib().ifattn_attention_state_blocks(self._h, None, 0, C.byref(n)))
        out = np.zeros(max(n.value, 1), np.int32)
        _check(lib().ifattn_attention_state_blocks(self._h, out.ctypes.data_as(C.POINTER(C.c_int32)),
                                                   out.size, C.byref(n)))
        return out[: n.value]

    def buffers(self) -> dict:
        b = StateBuffers()
        _check(lib().ifattn_attention_state_buffers_of(self._h, C.byref(b)))
        return {f: getattr(b, f) for f, _ in StateBuffers._fields_}

    def upload_table(self, stream=0) -> None:
        _check(lib().ifattn_attention_state_upload_table(self._h, stream))

    def set_length(self, kv_len: int, stream=0) -> None:
        _check(lib().ifattn_attention_state_set_length(self._h, kv_len, stream))

    def attend(self, window: int = 0, sinks: bool = False, stream=0) -> None:
        _check(lib().ifattn_attention_state_attend(self._h, window, int(sinks), stream))
