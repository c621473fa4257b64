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
    names = declared_functions() - {"inferfabric_kernel_v1"}
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
    assert not entry(1), "v1 must be refused: the operator needs I32/I64 or in-place tensors"
    k = entry(2).contents
    assert k.struct_bytes == C.sizeof(KernelV1) == 48  # 2 x u32, 2 strings, 3 function pointers
    assert k.abi_version == 2 and k.target == b"gfx950"
    assert k.contract.decode().startswith("inferfabric.") and k.contract.decode().endswith(".v2")


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
