"""The bench.py contract without a GPU: more than one GPU is refused with a
JSON message and exit status 2 before anything touches a device; the headline
traffic figure comes from the committed rocprofv3 summary and exceeds the
algorithmic bytes it is compared with; every secondary workload is named."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=str(ROOT))
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_traffic_comes_from_the_profile():
    import bench
    t = bench.measured_traffic()
    assert isinstance(t, int)
    # counter traffic of the config-2 decode kernel: at least its algorithmic
    # bytes (1878979976), and within a few percent of them
    assert 1878979976 <= t < 1.05 * 1878979976


def test_secondary_workloads_are_named():
    import bench
    assert {"c8_decode", "mla_decode", "mla_decode_c8", "mla_decode_rowq8", "mla_decode_rowq4",
            "mla_decode_step", "mixed_prefill_decode", "gated_attention_qwen",
            "mla_window_attention", "mla_sparse_attention", "slot_reuse",
            "norm_rope_write"} <= set(bench.SECONDARY)
