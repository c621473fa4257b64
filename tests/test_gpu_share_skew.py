"""GPU parity under the largest share skew the library accepts.

bf16 decode and dense bf16 MLA calls give odd workers smaller shares than
even ones (IFATTN_DECODE_XCD_SKEW / IFATTN_MLA_XCD_SKEW, permille of the
share, read once per process). At the extreme setting, and with one or three
workgroups per CU (even and odd persistent grids), every unit must still
belong to exactly one worker, so the decode and MLA parity cases of the other
test files are rerun in a child process with those settings. The MLA shares
of a CU's co-resident workgroups are also weighted by dispatch order
(IFATTN_MLA_SLOT_WEIGHTS); one run uses the most uneven weights accepted.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

TESTS = Path(__file__).resolve().parent

CASES = """
import sys
sys.path.insert(0, {tests!r})
import test_gpu_decode as d
import test_gpu_mla_attention as m
for shape in [(16, 2, 128, 128), (16, 2, 128, 32), (8, 8, 64, 32), (32, 2, 128, 64)]:
    d.test_decode_shapes(*shape)
d.test_decode_many_partitions()
d.test_decode_shares_slide_the_block_window()
d.test_decode_many_sequences()
d.test_decode_16_token_pages(128, False)
d.test_decode_step_matches_write_then_decode()
for seed in range(4):
    d.test_decode_random_shapes(seed)
d.test_decode_self_plan_limit(2, 513)
for rows in (1, 4, 16):
    m.test_window_ring_probe(rows)
for args in [(0, 64, False), (37, 64, True), (2500, 128, True)]:
    m.test_window_batches(*args)
m.test_many_rows(False, True, 300)
m.test_self_plan_row_limit(257, False)
m.test_dense_c8_weighted_shares(300)
m.test_dense_c8_weighted_shares(130)
m.test_sparse_batches(2048, 32, 128)
print("skew cases passed", flush=True)
"""


@pytest.mark.parametrize("wgs,weights", [("1", ""), ("3", ""), ("2", "1900,1000,100")])
def test_extreme_skew(wgs, weights):
    """The last case also gives the MLA dispatch slots the most uneven share
    weights accepted (none above twice the mean)."""
    env = dict(os.environ, IFATTN_DECODE_XCD_SKEW="200", IFATTN_MLA_XCD_SKEW="200",
               IFATTN_DECODE_WGS_PER_CU=wgs)
    if weights:
        env["IFATTN_MLA_SLOT_WEIGHTS"] = weights
    r = subprocess.run([sys.executable, "-c", CASES.format(tests=str(TESTS))], env=env,
                       capture_output=True, text=True, timeout=200)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "skew cases passed" in r.stdout
