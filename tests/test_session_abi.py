"""The session library libinferfabric_acl.so without a GPU: it exports exactly
the reference header's functions (native/include/inferfabric_acl.h), answers the
Rust loader's version check (crates/inferfabric-native/src/ffi.rs:40-45), fails
with a thread-local message where a caller breaks a rule, and names the entry
points it does not serve. Nothing here opens a session on a device."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "ironpangu_amd" / "libinferfabric_acl.so"


def session_lib():
    if not LIB.exists():
        pytest.fail("libinferfabric_acl.so is not built; run __graft_entry__.build()")
    l = C.CDLL(str(LIB))
    l.inferfabric_acl_last_error.restype = C.c_char_p
    l.inferfabric_acl_abi_version.restype = C.c_uint32
    l.inferfabric_acl_tp_root_size.restype = C.c_uint64
    return l


def declared(header):
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return {m.group(1) for m in re.finditer(r"\b(inferfabric_acl_[a-z_]+)\s*\(", text)}


def test_exports_exactly_the_declared_functions():
    names = declared(ROOT / "include" / "inferfabric_acl.h")
    assert len(names) == 38
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert names == exported


def test_version_and_rule_violations():
    l = session_lib()
    assert l.inferfabric_acl_abi_version() == 2
    assert l.inferfabric_acl_open(0, None) == -1
    assert b"null session output" in l.inferfabric_acl_last_error()
    # a null session is rejected before any device work, as the reference's guards do
    h = C.c_uint64(0)
    assert l.inferfabric_acl_allocate(None, C.c_uint64(16), C.byref(h)) == -1
    assert b"invalid allocation" in l.inferfabric_acl_last_error()
    assert l.inferfabric_acl_paged_attention_prepare(
        None, *([C.c_uint64(1)] * 10), C.c_int64(65), C.c_int64(24), C.c_int64(12),
        C.byref(h)) == -1
    assert b"invalid attention capacity" in l.inferfabric_acl_last_error()
    assert l.inferfabric_acl_attention_qk_prepare(
        None, *([C.c_uint64(1)] * 8), C.c_int64(0), C.byref(h)) == -1
    assert b"invalid QK batch" in l.inferfabric_acl_last_error()
    ids = (C.c_uint64 * 1)(1)
    assert l.inferfabric_acl_sequence_prepare(None, ids, C.c_uint64(1), C.byref(h)) == -1
    assert l.inferfabric_acl_close(None) == 0  # closing nothing succeeds, as the reference's
    assert l.inferfabric_acl_last_error() == b""


def test_unserved_entry_points_fail_by_name():
    l = session_lib()
    h = C.c_uint64(0)
    assert l.inferfabric_acl_linear_prepare(None, C.c_uint64(1), C.c_uint64(2), C.c_uint64(3),
                                            C.c_int64(1), C.c_int64(1), C.c_int64(1),
                                            C.byref(h)) == -1
    msg = l.inferfabric_acl_last_error()
    assert b"inferfabric_acl_linear_prepare: not in this library" in msg
    assert l.inferfabric_acl_rms_prepare(None, C.c_uint64(1), C.c_uint64(2), C.c_uint64(3),
                                         C.c_int64(1), C.c_int64(1), C.byref(h)) == -1
    assert b"rms_prepare: not in this library" in l.inferfabric_acl_last_error()
    assert l.inferfabric_acl_tp_root_size() == 0
    assert l.inferfabric_acl_tp_root(None, C.c_uint64(0)) == -1


def test_error_text_is_per_thread():
    import threading
    l = session_lib()
    assert l.inferfabric_acl_open(0, None) == -1
    seen = {}

    def other():
        seen["msg"] = l.inferfabric_acl_last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == b""
    assert b"null session output" in l.inferfabric_acl_last_error()
