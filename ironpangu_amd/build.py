"""Build recipe for the gfx950 shared library ``libifattn_hip.so``.

Every ``csrc/*.hip`` file is compiled for gfx950 with hipcc and every
``csrc/*.cpp`` file as host C++, in parallel, into ``_build/``; the objects
are linked into ``ironpangu_amd/libifattn_hip.so`` next to this file. The
IFKernelV1 plug-in shims (one ``libifk_<name>.so`` per operator contract) and
the session-ABI library ``libinferfabric_acl.so`` are linked against it with an
``$ORIGIN`` rpath.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libifattn_hip.so"
SESSION_LIB = PKG / "libinferfabric_acl.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Wno-unused-function", "-Wno-unused-variable",
    # Keep hipcc from forming packed fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]
HOST_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__"]
# Attention kernels: no NaN semantics for fmaxf (otherwise every operand is
# canonicalized with an extra v_max_f32 before each max in the softmax).
# Outputs for NaN inputs are unspecified by the operator contracts.
FILE_FLAGS = {
    "varlen_prefill.hip": ["-fno-honor-nans"],
}

# IFKernelV1 contracts exported as separate plug-in libraries (name -> contract index).
PLUGINS = {
    "kv_cache_write_bf16": 0,
    "kv_cache_write_c8": 1,
    "paged_decode_gqa_bf16": 2,
    "paged_decode_gqa_c8": 3,
    "varlen_prefill_bf16": 4,
    "mla_decode_bf16": 5,
    "mla_decode_c8": 6,
    "mla_cache_write_c8": 7,
    "mla_norm_rope_cache_bf16": 8,
    "mla_norm_rope_cache_c8": 9,
    "mla_window_attention_w512_bf16": 10,
    "mla_window_attention_w2048_bf16": 11,
    "mla_sparse_attention_c8": 12,
    "paged_attention_qwen_gated_bf16": 13,
}


def _hipcc() -> str:
    p = ROCM / "bin" / "hipcc"
    return str(p) if p.exists() else "hipcc"


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        noise = "packed-fp32-ops' is not a recognized feature"
        err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{err}")


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [_hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *HOST_FLAGS, f"-I{ROCM}/include", "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build(jobs: int | None = None, plugins: bool = True) -> Path:
    """Compile every source and link ``libifattn_hip.so``; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(
        p for p in CSRC.glob("*.cpp") if p.name != "plugin_shim.cpp")
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    shutil.move(str(tmp), LIB)
    shim = CSRC / "plugin_shim.cpp"
    if plugins and shim.exists():
        def one(item):
            name, idx = item
            out = PKG / f"libifk_{name}.so"
            _run(["g++", *HOST_FLAGS, "-shared", f"-DIFK_CONTRACT_INDEX={idx}", str(shim),
                  f"-L{PKG}", "-lifattn_hip", "-Wl,-rpath,$ORIGIN", "-o", str(out)])
        with cf.ThreadPoolExecutor(jobs) as ex:
            list(ex.map(one, PLUGINS.items()))
    session = PKG / "session" / "inferfabric_acl.cpp"
    if session.exists():  # the reference's session ABI, over libifattn_hip.so
        exports = BUILD / "inferfabric_acl.map"  # export the ABI's symbols only
        exports.write_text("{ global: inferfabric_acl_*; local: *; };\n")
        _run(["g++", *HOST_FLAGS, f"-Wl,--version-script={exports}", f"-I{ROCM}/include",
              "-shared", str(session), f"-L{PKG}",
              "-lifattn_hip", f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN",
              f"-Wl,-rpath,{ROCM}/lib", "-o", str(SESSION_LIB)])
    driver = CSRC.parent / "driver" / "ifattn_drive.cpp"
    if driver.exists():
        _run(["g++", *HOST_FLAGS, f"-I{ROCM}/include", str(driver), f"-L{ROCM}/lib",
              "-lamdhip64", "-ldl", f"-Wl,-rpath,{ROCM}/lib", "-o", str(PKG / "ifattn_drive")])
    return LIB


if __name__ == "__main__":
    print(build())
