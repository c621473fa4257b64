"""C-ABI boundary checks that need no GPU: the library loads and exports every
function declared under include/, the per-operator IFKernelV1 plug-ins answer
the reference loader's handshake, and prepare validates descriptors (shapes,
dtypes, access, contiguity, aliasing) without touching the device."""
import ctypes as C
import re
from pathlib import Path

import pytest

from ironpangu_amd import _native
from ironpangu_amd.build import PLUGINS

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if name.startswith(("ifattn_", "if_", "inferfabric_")) and not name.endswith("_t"):
                names.add(name)
    return names


def test_library_exports_every_declared_function():
    lib = _native.lib()
    # inferfabric_acl_* is the session library's (tests/test_session_abi.py).
    names = {n for n in declared_functions() - {"inferfabric_kernel_v1"}
             if not n.startswith("inferfabric_acl_")}
    assert len(names) >= 30
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.ifattn_abi_version() == 1


def test_host_errors_without_device():
    lib = _native.lib()
    st = lib.ifattn_paged_decode_bf16(None, None, None, None, 1, None, None, 1, 16, 2, 128, 128,
                                      1, 128, 0.1, None, 0, None)
    assert st == -1 and b"null" in lib.ifattn_last_error()
    st = lib.ifattn_kv_cache_write(1, 2, 3, 4, 5, 7, 1, 1024, 10, None)  # bad slot dtype
    assert st == -1 and b"dtype" in lib.ifattn_last_error()
    assert lib.ifattn_paged_decode_workspace_size(256, 16, 128, 256) > 64
    assert lib.ifattn_mla_decode_workspace_size(0, 16, 64, 64) == 0


class Tensor(C.Structure):
    _fields_ = [("struct_bytes", C.c_uint32), ("dtype", C.c_uint32), ("rank", C.c_uint32),
                ("access", C.c_uint32), ("data", C.c_void_p), ("allocation_bytes", C.c_uint64),
                ("shape", C.c_int64 * 8), ("strides", C.c_int64 * 8)]


class Prepared(C.Structure):
    _fields_ = [("state", C.c_void_p), ("workspace_bytes", C.c_uint64),
                ("workspace_alignment", C.c_uint64)]


PREPARE = C.CFUNCTYPE(C.c_int32, C.POINTER(Tensor), C.c_uint32, C.POINTER(Tensor), C.c_uint32,
                      C.POINTER(Prepared))
ENQUEUE = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p)
RELEASE = C.CFUNCTYPE(None, C.c_void_p)


class KernelV1(C.Structure):
    _fields_ = [("struct_bytes", C.c_uint32), ("abi_version", C.c_uint32),
                ("contract", C.c_char_p), ("target", C.c_char_p), ("prepare", PREPARE),
                ("enqueue", ENQUEUE), ("release", RELEASE)]


ESIZE = {1: 1, 2: 2, 3: 4, 4: 4, 5: 8}
_fake = [0x100000]


def tensor(shape, dtype, access, addr=None):
    t = Tensor()
    t.struct_bytes = C.sizeof(Tensor)
    t.dtype, t.rank, t.access = dtype, len(shape), access
    n = 1
    for s in shape:
        n *= s
    if addr is None:  # distinct fake addresses: prepare never dereferences them
        addr = _fake[0]
        _fake[0] += (n * ESIZE[dtype] + 4095) // 4096 * 4096 + 4096
    t.data = addr
    t.allocation_bytes = n * ESIZE[dtype]
    stride = 1
    for i in reversed(range(len(shape))):
        t.shape[i] = shape[i]
        t.strides[i] = stride
        stride *= shape[i]
    return t


def load_plugin(name):
    _native.lib()  # load the main library first (RTLD_GLOBAL)
    so = C.CDLL(str(ROOT / "ironpangu_amd" / f"libifk_{name}.so"))
    entry = so.inferfabric_kernel_v1
    entry.restype = C.POINTER(KernelV1)
    entry.argtypes = [C.c_uint32]
    return so, entry


@pytest.mark.parametrize("name", sorted(PLUGINS))
def test_plugin_handshake(name):
    so, entry = load_plugin(name)
    k = entry(2).contents
    assert k.struct_bytes == C.sizeof(KernelV1) == 48  # 2 x u32, 2 strings, 3 function pointers
    assert k.abi_version == 2 and k.target == b"gfx950"
    assert k.contract.decode().startswith("inferfabric.") and k.contract.decode().endswith(".v2")
    assert not entry(0) and not entry(3)
    if name == "paged_attention_qwen_gated_bf16":
        assert not entry(1), "reads the caches it appends to: no version-1 form"
        return
    k1 = entry(1).contents
    assert k1.abi_version == 1 and k1.target == b"gfx950"
    assert k1.contract.decode() == k.contract.decode()[:-3] + ".v1"


def _prepare(k, ins, outs):
    a = (Tensor * len(ins))(*ins)
    b = (Tensor * len(outs))(*outs)
    p = Prepared()
    st = k.prepare(a, len(ins), b, len(outs), C.byref(p))
    return st, p


def decode_ports(n=4, hq=16, hkv=2, d=128, nb=64, bs=128, entries=8):
    q = tensor([n, hq, d], 2, 1)
    kc = tensor([nb, bs, hkv, d], 2, 1)
    vc = tensor([nb, bs, hkv, d], 2, 1)
    bt = tensor([n, entries], 4, 1)
    sl = tensor([n], 4, 1)
    out = tensor([n, hq, d], 2, 2)
    return [q, kc, vc, bt, sl], [out]


def test_decode_prepare_and_rejections():
    so, entry = load_plugin("paged_decode_gqa_bf16")
    k = entry(2).contents
    ins, outs = decode_ports()
    st, p = _prepare(k, ins, outs)
    assert st == 0 and p.state and p.workspace_alignment == 256
    assert p.workspace_bytes == _native.lib().ifattn_paged_decode_workspace_size(4, 16, 128, 1024)
    k.release(p.state)
    bad = decode_ports()
    bad[0][3].dtype = 5  # I64 block tables
    assert _prepare(k, *bad)[0] != 0
    bad = decode_ports()
    bad[0][0].strides[0] = 9999  # non-contiguous
    st, p = _prepare(k, *bad)
    assert st != 0 and not p.state
    bad = decode_ports()
    bad[1][0].data = bad[0][0].data  # output aliases q
    assert _prepare(k, *bad)[0] != 0
    bad = decode_ports()
    bad[1][0].access = 1
    assert _prepare(k, *bad)[0] != 0
    bad = decode_ports()
    bad[0][1].shape[3] = 64  # cache head_dim mismatch (strides now wrong too)
    assert _prepare(k, *bad)[0] != 0


def test_write_and_mla_prepare():
    so, entry = load_plugin("kv_cache_write_c8")
    k = entry(2).contents
    ins = [tensor([8, 2, 128], 2, 1), tensor([8, 2, 128], 2, 1), tensor([8], 5, 1)]
    outs = [tensor([4, 32, 2, 128], 1, 3), tensor([4, 32, 2, 128], 1, 3),
            tensor([4, 32, 2], 3, 3), tensor([4, 32, 2], 3, 3)]
    st, p = _prepare(k, ins, outs)
    assert st == 0 and p.workspace_bytes == 0
    k.release(p.state)
    outs[3] = tensor([4, 32, 1], 3, 3)
    assert _prepare(k, ins, outs)[0] != 0
    so, entry = load_plugin("mla_decode_c8")
    k = entry(2).contents
    ins = [tensor([4, 16, 576], 2, 1), tensor([32, 64, 656], 1, 1), tensor([4, 16], 4, 1),
           tensor([4], 4, 1)]
    outs = [tensor([4, 16, 512], 2, 2)]
    st, p = _prepare(k, ins, outs)
    assert st == 0 and p.workspace_bytes == _native.lib().ifattn_mla_decode_workspace_size(4, 16, 1024, 64)
    k.release(p.state)
    ins[1] = tensor([32, 64, 576], 1, 1)
    assert _prepare(k, ins, outs)[0] != 0


def test_norm_rope_write_prepare():
    so, entry = load_plugin("mla_norm_rope_cache_c8")
    k = entry(2).contents
    assert k.contract == b"inferfabric.mla_norm_rope_cache.c8.v2"

    def ports(rows=17, width=656, cache_dtype=1, cos_rows=None):
        ins = [tensor([rows, 576], 2, 1), tensor([512], 2, 1),
               tensor([cos_rows or rows, 64], 2, 1), tensor([cos_rows or rows, 64], 2, 1),
               tensor([rows], 5, 1)]
        return ins, [tensor([256, 32, width], cache_dtype, 3)]

    st, p = _prepare(k, *ports())
    assert st == 0 and p.state and p.workspace_bytes == 0
    k.release(p.state)
    assert _prepare(k, *ports(width=576))[0] != 0        # c8 rows are 656 bytes
    assert _prepare(k, *ports(cos_rows=3))[0] != 0       # cos/sin per row
    assert _prepare(k, *ports(rows=4097))[0] != 0        # the reference's 4096-row bound
    so, entry = load_plugin("mla_norm_rope_cache_bf16")
    k = entry(2).contents
    st, p = _prepare(k, *ports(width=576, cache_dtype=2))
    assert st == 0
    k.release(p.state)


def test_mla_attention_prepare():
    so, entry = load_plugin("mla_sparse_attention_c8")
    k = entry(2).contents

    def ports(rows=5, heads=6, topk=512, sinks=128, width=656):
        ins = [tensor([rows, heads, 576], 2, 1), tensor([64, 32, width], 1, 1),
               tensor([rows, topk], 4, 1), tensor([2, 32], 4, 1), tensor([3], 4, 1),
               tensor([2], 4, 1), tensor([sinks, 576], 2, 1), tensor([sinks, 512], 2, 1)]
        return ins, [tensor([rows, heads, 512], 2, 2)]

    st, p = _prepare(k, *ports())
    lib = _native.lib()
    assert st == 0 and p.workspace_bytes == lib.ifattn_mla_attention_workspace_size(5, 6, 1024, 0, 512, 128, 32)
    k.release(p.state)
    assert _prepare(k, *ports(sinks=129))[0] != 0     # at most 128 sink rows
    assert _prepare(k, *ports(width=576))[0] != 0     # C8 rows are 656 bytes
    assert _prepare(k, *ports(heads=17))[0] != 0
    so, entry = load_plugin("mla_window_attention_w2048_bf16")
    k = entry(2).contents
    ins = [tensor([4, 16, 576], 2, 1), tensor([64, 16, 576], 2, 1), tensor([1, 4096], 4, 1),
           tensor([2], 4, 1), tensor([1], 4, 1), tensor([128, 576], 2, 1), tensor([128, 512], 2, 1)]
    st, p = _prepare(k, ins, [tensor([4, 16, 512], 2, 2)])
    assert st == 0
    assert p.workspace_bytes == lib.ifattn_mla_attention_workspace_size(4, 16, 65536, 2048, 0, 128, 16)
    k.release(p.state)


def test_work_item_encoding_bounds():
    """Decode and prefill work items pack (sequence << 12 | tile) in 32 bits:
    2^20 sequences, or more than 4096 query tiles per sequence, are refused on
    the host (fake device addresses: nothing is launched)."""
    lib = _native.lib()
    a = 0x10000
    st = lib.ifattn_paged_decode_bf16(a, a, a, a, 8, a, a, 1 << 20, 16, 2, 128, 128, 8, 1024,
                                      0.1, a, 1 << 40, None)
    assert st == -1 and b"2^20" in lib.ifattn_last_error()
    st = lib.ifattn_varlen_prefill_bf16(a, a, a, a, 8, a, a, a, 1 << 20, 1 << 20, 1, 1024, 16, 2,
                                        128, 128, 8, 0.1, a, 1 << 40, None)
    assert st == -1 and b"2^20" in lib.ifattn_last_error()
    # head_dim 256, group 16: 8-row query tiles, so 4096 tiles hold 32768 rows
    st = lib.ifattn_varlen_prefill_bf16(a, a, a, a, 2048, a, a, a, 1, 32769, 32769, 262144, 16, 1,
                                        256, 128, 2048, 0.1, a, 1 << 40, None)
    assert st == -1 and b"4096 query tiles" in lib.ifattn_last_error()


# ---- the reference's own loader (native/src/compiled_kernel.cpp, compiled in place)

def _ref_loader():
    import oracle
    l = oracle.ref_loader()
    if l is None:
        pytest.skip("reference loader not built (reference tree absent at build time)")
    return l


def ref_open(name, contract):
    l = _ref_loader()
    _native.lib()
    h = C.c_void_p()
    st = l.ref_loader_open(str(ROOT / "ironpangu_amd" / f"libifk_{name}.so").encode(),
                           contract.encode(), b"gfx950", C.byref(h))
    return st, h, l


def ref_prepare(l, h, ins, outs):
    a = (Tensor * len(ins))(*ins)
    b = (Tensor * len(outs))(*outs)
    p, ws = C.c_void_p(), C.c_uint64()
    st = l.ref_loader_prepare(h, C.cast(a, C.c_void_p), len(ins), C.cast(b, C.c_void_p), len(outs),
                              C.byref(p), C.byref(ws))
    return st, p, ws.value


def byte_view(shape, width):
    """Version-1 integer port: I8 tensor whose last extent is width x the count."""
    return tensor(list(shape[:-1]) + [shape[-1] * width], 1, 1)


@pytest.mark.parametrize("name", sorted(set(PLUGINS) - {"paged_attention_qwen_gated_bf16"}))
def test_reference_loader_accepts_every_v1_plugin(name):
    so, entry = load_plugin(name)
    contract = entry(1).contents.contract.decode()
    st, h, l = ref_open(name, contract)
    assert st == 0, l.ref_loader_error()
    l.ref_loader_close(h)
    # the v2 name is not what version 1 answers
    st, h, l = ref_open(name, contract[:-3] + ".v2")
    assert st != 0 and b"contract" in l.ref_loader_error()


def test_reference_loader_prepares_v1_decode_and_write():
    st, h, l = ref_open("paged_decode_gqa_bf16", "inferfabric.paged_decode.gqa.bf16.v1")
    assert st == 0
    n, hq, hkv, d, nb, bs, entries = 4, 16, 2, 128, 64, 128, 8
    ins = [tensor([n, hq, d], 2, 1), tensor([nb, bs, hkv, d], 2, 1), tensor([nb, bs, hkv, d], 2, 1),
           byte_view([n, entries], 4), byte_view([n], 4)]
    outs = [tensor([n, hq, d], 2, 2)]
    st, p, ws = ref_prepare(l, h, ins, outs)
    assert st == 0, l.ref_loader_error()
    assert ws == _native.lib().ifattn_paged_decode_workspace_size(n, hq, d, entries * bs)
    l.ref_loader_release(p)
    # an I32 dtype is outside version 1: the reference loader itself refuses it
    bad = list(ins)
    bad[3] = tensor([n, entries], 4, 1)
    assert ref_prepare(l, h, bad, outs)[0] != 0 and b"dtype" in l.ref_loader_error()
    # a byte view whose length is not whole int32s: the plug-in refuses it
    bad = list(ins)
    bad[4] = tensor([n * 4 + 1], 1, 1)
    assert ref_prepare(l, h, bad, outs)[0] != 0
    l.ref_loader_close(h)
    # in-place cache write: caches are write-only outputs in version 1
    st, h, l = ref_open("kv_cache_write_c8", "inferfabric.kv_cache_write.c8.v1")
    ins = [tensor([8, 2, 128], 2, 1), tensor([8, 2, 128], 2, 1), byte_view([8], 8)]
    outs = [tensor([4, 32, 2, 128], 1, 2), tensor([4, 32, 2, 128], 1, 2),
            tensor([4, 32, 2], 3, 2), tensor([4, 32, 2], 3, 2)]
    st, p, ws = ref_prepare(l, h, ins, outs)
    assert st == 0 and ws == 0, l.ref_loader_error()
    l.ref_loader_release(p)
    l.ref_loader_close(h)
