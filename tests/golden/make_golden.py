"""Writes tests/golden/host_meta.json: input/output vectors of the reference's
own host metadata code (native/src/page_binding.h, native/include/sequence_batch.h),
compiled in place from /root/reference into oracle/_ref/libref_meta.so
(`make -C oracle ref`). Run in a container where the reference tree exists:
    python tests/golden/make_golden.py
The fixture lets the product be checked against the reference where the
reference tree (and so the _ref build) is absent.
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "host_meta.json"


def ref():
    r = oracle.ref()
    if r is None:
        raise SystemExit("oracle/_ref/libref_meta.so is not built (needs /root/reference)")
    return r


def p32(a):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


class RefPages:
    def __init__(self, page, logical, slots, shared):
        self.r = ref()
        self.h = C.c_void_p()
        st = self.r.ref_pages_create(C.c_uint32(page), C.c_uint32(logical), C.c_uint32(slots),
                                     C.c_int(int(shared)), C.byref(self.h))
        assert st == 0

    def call(self, name, *args):
        return getattr(self.r, name)(self.h, *args)

    def bind(self, pages):
        a = np.ascontiguousarray(pages, np.int32)
        return self.call("ref_pages_bind", p32(a), C.c_uint64(a.size))

    def select(self, s):
        return self.call("ref_pages_select", C.c_uint32(s))

    def release(self, s):
        return self.call("ref_pages_release", C.c_uint32(s))

    def append(self, slot, pos):
        out = C.c_uint64()
        st = self.call("ref_pages_append", C.c_uint32(slot), C.c_uint32(pos), C.byref(out))
        return None if st else int(out.value)

    def batch_table(self, residents, entries, ring):
        a = np.ascontiguousarray(residents, np.int32)
        out = np.zeros(max(a.size * entries, 1), np.int32)
        st = self.call("ref_pages_batch_table", p32(a), C.c_uint64(a.size), C.c_uint32(entries),
                       C.c_int(int(ring)), p32(out))
        return None if st else out[: a.size * entries].tolist()

    def copy_plan(self, src, dst, completed, windowed, field):
        buf = np.zeros(3 * 4096, np.uint64)
        n = C.c_uint64()
        st = self.call("ref_pages_copy_plan", C.c_uint32(src), C.c_uint32(dst),
                       C.c_uint32(completed), C.c_int(int(windowed)), C.c_uint64(field),
                       buf.ctypes.data_as(C.POINTER(C.c_uint64)), C.c_uint64(4096), C.byref(n))
        return None if st else [buf[3 * i:3 * i + 3].tolist() for i in range(n.value)]


def ref_spans(pages, page_bytes, field):
    a = np.ascontiguousarray(pages, np.int32)
    buf = np.zeros(2 * 8192, np.uint64)
    n = C.c_uint64()
    st = ref().ref_page_spans(p32(a) if a.size else None, C.c_uint64(a.size), C.c_uint64(page_bytes),
                              C.c_uint64(field), buf.ctypes.data_as(C.POINTER(C.c_uint64)),
                              C.c_uint64(8192), C.byref(n))
    return None if st else [buf[2 * i:2 * i + 2].tolist() for i in range(n.value)]


class Slice(C.Structure):
    _fields_ = [("resident", C.c_uint32), ("position", C.c_uint32), ("tokens", C.c_uint32),
                ("sample", C.c_int32)]


def ref_batch(seqs, cap, budget, context):
    n = len(seqs)
    arr = (Slice * max(n, 1))(*[Slice(*s) for s in seqs])
    total = sum(s[2] for s in seqs)
    rows_cap = max(min(total, 1 << 20), 1)
    bufs = [np.zeros(max(k, 1), dt) for k, dt in
            [(n + 1, np.int32), (n, np.int32), (n, np.int32), (n, np.int32), (n, np.int32),
             (rows_cap, np.int32), (rows_cap, np.int32), (rows_cap, np.int64), (n, np.uint32),
             (n, np.uint32)]]
    rows, samples = C.c_uint64(), C.c_uint64()
    st = ref().ref_sequence_batch(arr, C.c_uint64(n), C.c_uint32(cap), C.c_uint32(budget),
                                  C.c_uint32(context), C.c_uint64(rows_cap),
                                  *[b.ctypes.data_as(C.c_void_p) for b in bufs],
                                  C.byref(rows), C.byref(samples))
    if st:
        return None
    r, s = rows.value, samples.value
    names = ["starts", "query_ends", "prior_lengths", "kv_lengths", "residents", "positions",
             "row_residents", "lengths", "sample_rows", "sample_residents"]
    lens = [n + 1, n, n, n, n, r, r, r, s, s]
    return {k: b[:m].tolist() for k, b, m in zip(names, bufs, lens)}


def main():
    rng = np.random.default_rng(20261201)
    cases = []
    # 1. fragmented fixed bindings + slot mapping + batch tables (fixed and ring)
    for page, logical, slots in [(16, 512, 4), (32, 1024, 3), (128, 4096, 8), (64, 2048, 2)]:
        rp = RefPages(page, logical, slots, False)
        ops = []
        per = logical // page
        for s in range(slots):
            perm = (s * per + rng.permutation(per)).astype(np.int32).tolist()
            rp.select(s)
            ops.append(["select", s, 0])
            ops.append(["bind", perm, rp.bind(perm)])
        bad = list(range(per))
        bad[0] = bad[1]
        ops.append(["bind", bad, rp.bind(bad)])  # alias: rejected
        rows = [(int(rng.integers(slots)), int(rng.integers(logical))) for _ in range(64)]
        appends = [rp.append(s, q) for s, q in rows]
        residents = rng.permutation(slots)[: max(1, slots - 1)].astype(np.int32).tolist()
        cases.append({"kind": "fixed", "page": page, "logical": logical, "slots": slots,
                      "ops": ops, "rows": rows, "appends": appends, "residents": residents,
                      "table": rp.batch_table(residents, per, False),
                      "ring": rp.batch_table(residents, per * 2 + 1, True)})
    # 2. shared reservations with partial claims, rejections and releases
    for page, logical, slots in [(16, 256, 4), (32, 1024, 3)]:
        rp = RefPages(page, logical, slots, True)
        per = logical // page
        pool = per * slots
        ops = []
        for s in range(slots):
            ops.append(["release", s, rp.release(s)])
        for step in range(24):
            s = int(rng.integers(slots))
            ops.append(["select", s, rp.select(s)])
            k = int(rng.integers(1, per + 1))
            pages = rng.choice(pool, size=k, replace=False).astype(np.int32).tolist()
            ops.append(["bind", pages, rp.bind(pages)])
            if step % 5 == 4:
                r = int(rng.integers(slots))
                ops.append(["release", r, rp.release(r)])
        rows = [(int(rng.integers(slots)), int(rng.integers(logical))) for _ in range(64)]
        appends = [rp.append(s, q) for s, q in rows]
        cases.append({"kind": "shared", "page": page, "logical": logical, "slots": slots,
                      "ops": ops, "rows": rows, "appends": appends,
                      "table": rp.batch_table(list(range(slots)), per, False),
                      "copy": [[a, b, c, w, f, rp.copy_plan(a, b, c, w, f)] for a, b, c, w, f in
                               [(0, 1, page, False, pool * page * 4), (1, 2, 2 * page, True, pool * 7),
                                (2, 0, logical, False, pool * 2), (0, 1, page + 1, False, pool)]]})
    # 3. page spans
    spans = []
    for page_bytes in (2, 128, 656, 1152):
        for pages in ([], [4, 0, 3, 1, 8], [9], rng.permutation(10)[:6].tolist(), [3, 3], [10]):
            spans.append([pages, page_bytes, 10 * page_bytes,
                          ref_spans(pages, page_bytes, 10 * page_bytes)])
    # 4. sequence batches (valid and rejected)
    batches = []
    for trial in range(30):
        n = int(rng.integers(1, 6))
        cap = int(rng.integers(n, n + 4))
        res = rng.permutation(cap)[:n].tolist()
        if trial % 7 == 3:
            res[-1] = res[0]  # duplicate resident
        seqs = [(int(r), int(rng.integers(0, 600)), int(rng.integers(0 if trial % 11 == 5 else 1, 300)),
                 int(rng.integers(2))) for r in res]
        budget = int(rng.integers(200, 1600))
        context = int(rng.integers(400, 1000))
        batches.append([seqs, cap, budget, context, ref_batch(seqs, cap, budget, context)])
    OUT.write_text(json.dumps({"source": "reference host metadata compiled in place (oracle/_ref)",
                               "pages": cases, "spans": spans, "batches": batches}))
    print("wrote", OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
