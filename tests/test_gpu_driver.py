"""The stand-alone C++ driver (ironpangu_amd/driver/ifattn_drive.cpp): no Python
in the process, libifattn_hip.so and the IFKernelV1 plug-ins bound with dlopen,
host metadata through the host C ABI, device memory through hipMalloc. It runs the
fused decode step directly and the write + decode plug-ins on a copy of the same
caches, and reports whether outputs and caches agree bit for bit.
"""
import json
import subprocess
from pathlib import Path

import pytest

DRIVER = Path(__file__).resolve().parents[1] / "ironpangu_amd" / "ifattn_drive"


@pytest.mark.gpu
@pytest.mark.parametrize("seqs,lo,hi,seed", [(1, 1, 1, 3), (8, 16, 512, 1), (64, 100, 4096, 7)])
def test_driver_plugin_equals_direct(seqs, lo, hi, seed):
    if not DRIVER.exists():
        pytest.fail("ifattn_drive is not built; run __graft_entry__.build()")
    print(f"driver seqs={seqs} lens=[{lo},{hi}] seed={seed}", flush=True)
    r = subprocess.run([str(DRIVER), "--seqs", str(seqs), "--lo", str(lo), "--hi", str(hi),
                        "--seed", str(seed), "--steps", "5"],
                       capture_output=True, text=True, timeout=90)
    line = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else ""
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    rep = json.loads(line)
    assert rep["status"] == "ok"
    assert all(rep["plugin_equals_direct"].values())
    assert rep["ms_per_step"] > 0


def test_driver_rejects_bad_arguments():
    if not DRIVER.exists():
        pytest.skip("ifattn_drive is not built")
    r = subprocess.run([str(DRIVER), "--seqs", "0"], capture_output=True, text=True, timeout=30)
    assert r.returncode == 1
    assert json.loads(r.stdout.strip())["status"] == "error"
