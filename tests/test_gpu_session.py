"""The session ABI on the GPU.

1. The q/k producer kernel (ifattn_qk_norm_rope_gate_bf16) against
   oracle_qk_norm_rope_gate on random heads and positions.
2. tests/native/acl_session_probe (a C++ process with no Python in it) replays
   the reference's Qwen attention probe call sequence
   (crates/inferfabric-cli/src/npu_probe/attention.rs:82-200) through
   libinferfabric_acl.so: qk prepare + paged attention prepare + sequence,
   capture, then per token execute and replay with rewritten append rows,
   tables and masks. It requires replay == eager bit for bit and dumps the
   eager results; here each token is recomputed with the oracle:
   * appended V rows bit-exact, appended K rows equal to the oracle's
     normed/rotated k (bf16, at most one ulp apart);
   * every other cache row unchanged;
   * outputs within 1e-2 abs + 1e-2 rel and relative L2 <= 0.02 (the
     reference probe's bound, attention.rs:269).
   Run at the reference probe's shape and at a larger one (64 requests, 1000
   prior positions, 16-token pages) that takes the split-context path.
"""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import assert_close

ROOT = Path(__file__).resolve().parent.parent
PROBE = ROOT / "tests" / "native" / "acl_session_probe"
LIB = ROOT / "ironpangu_amd" / "libinferfabric_acl.so"


def bf16_val(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def ulp_diff(a, b):
    """|a - b| in bf16 ulps for finite bf16 bit patterns (sign-magnitude order)."""
    def order(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + x)
    return np.abs(order(a) - order(b))


@pytest.mark.gpu
@pytest.mark.parametrize("batch,seed", [(1, 0), (7, 1), (64, 2)])
def test_qk_kernel_matches_oracle(batch, seed):
    import torch
    from ironpangu_amd import ops
    from helpers import bits_host, to_dev
    print(f"qk kernel batch={batch} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    pq = bf16_bits(rng.standard_normal((batch, 8, 512)) * 1.5)
    k = bf16_bits(rng.standard_normal((batch, 2, 256)) * 0.6)
    qg = (bf16_val(bf16_bits(rng.uniform(-0.4, 0.4, 256))) + 1).astype(np.float32)
    kg = (bf16_val(bf16_bits(rng.uniform(-0.4, 0.4, 256))) + 1).astype(np.float32)
    pos = rng.integers(0, 262144, batch).astype(np.int64)
    pos[0] = 0
    q, ko, gate = ops.qk_norm_rope_gate(to_dev(pq), to_dev(k), to_dev(qg), to_dev(kg), to_dev(pos))
    torch.cuda.synchronize()
    eq, ek, eg = oracle.qk_norm_rope_gate(pq, k, qg, kg, pos)
    for got, exp, name in ((bits_host(q), eq, "q"), (bits_host(ko), ek, "k"),
                           (bits_host(gate), eg, "gate")):
        d = ulp_diff(got, exp)
        assert d.max() <= 1, (name, int(d.max()))
        assert (d == 0).mean() > 0.995, (name, float((d == 0).mean()))


def run_probe(tmp_path, *args):
    if not PROBE.exists() or not LIB.exists():
        pytest.fail("session library or probe not built; run __graft_entry__.build()")
    dump = tmp_path / "session.bin"
    print("acl_session_probe", *args, flush=True)
    r = subprocess.run([str(PROBE), "--lib", str(LIB), "--dump", str(dump), *args],
                       capture_output=True, text=True, timeout=100, cwd=str(ROOT))
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    rep = json.loads(r.stdout.strip().splitlines()[-1])
    assert rep["status"] == "ok" and rep["abi_version"] == 2
    assert rep["graph_equals_eager"] is True
    assert rep["linear_refused"] is True
    return rep, dump


def check_dump(rep, dump, initial_rows):
    B, C, S, T = rep["batch"], rep["context"], rep["slots"], rep["tokens"]
    raw = dump.read_bytes()
    off = 0

    def take(dtype, n):
        nonlocal off
        a = np.frombuffer(raw, dtype, n, off)
        off += a.nbytes
        return a

    qgamma, kgamma = take(np.float32, 256), take(np.float32, 256)
    keys = initial_rows(S).copy()
    values = keys.copy()
    written = np.zeros(S, bool)
    for t in range(T):
        qin = take(np.uint16, B * 4096).reshape(B, 8, 512)
        kin = take(np.uint16, B * 512).reshape(B, 2, 256)
        vin = take(np.uint16, B * 512).reshape(B, 512)
        pos = take(np.int64, B)
        idx = take(np.int64, B)
        table = take(np.int64, B * C).reshape(B, C)
        mask = take(np.float32, B * C).reshape(B, C)
        out = take(np.uint16, B * 2048).reshape(B, 8, 256)
        rows = take(np.uint16, B * 1024).reshape(B, 2, 512)
        eq, ek, eg = oracle.qk_norm_rope_gate(qin, kin, qgamma, kgamma, pos)
        assert np.array_equal(rows[:, 1], vin), f"token {t}: appended V rows differ"
        d = ulp_diff(rows[:, 0], ek.reshape(B, 512))
        assert d.max() <= 1, f"token {t}: appended K rows off by {int(d.max())} ulp"
        keys[idx] = ek.reshape(B, 512)
        values[idx] = vin
        written[idx] = True
        exp = oracle.gated_attention(eq, keys, values, table, mask, eg)
        got = bf16_val(out)
        assert_close(got, exp, what=f"token {t} output")
        rel = np.sqrt(((got - exp) ** 2).sum() / max((exp.astype(np.float64) ** 2).sum(), 1e-20))
        assert rel <= 0.02, (t, rel)
    fk = take(np.uint16, S * 512).reshape(S, 512)
    fv = take(np.uint16, S * 512).reshape(S, 512)
    assert off == len(raw)
    base = initial_rows(S)
    assert np.array_equal(fk[~written], base[~written]), "untouched K rows changed"
    assert np.array_equal(fv[~written], base[~written]), "untouched V rows changed"
    assert np.array_equal(fv[written], values[written])
    assert ulp_diff(fk[written], keys[written]).max() <= 1


@pytest.mark.gpu
def test_session_probe_reference_sequence(tmp_path):
    rep, dump = run_probe(tmp_path)
    assert (rep["batch"], rep["context"], rep["slots"], rep["page"], rep["tokens"]) == (2, 12, 24, 4, 6)
    check_dump(rep, dump, lambda s: np.full((s, 512), bf16_bits(np.float32(0.75)), np.uint16))


def pattern_rows(slots):
    slot = np.arange(slots, dtype=np.int64)[:, None]
    col = np.arange(512, dtype=np.int64)[None, :]
    v = ((slot * 131 + col * 7) % 97).astype(np.float32) / np.float32(48) - np.float32(1)
    return bf16_bits(v)


@pytest.mark.gpu
def test_session_probe_split_context(tmp_path):
    rep, dump = run_probe(tmp_path, "--batch", "64", "--context", "1024", "--prior", "1000",
                          "--page", "16", "--slots", "65536", "--tokens", "3", "--seed", "5")
    check_dump(rep, dump, pattern_rows)
