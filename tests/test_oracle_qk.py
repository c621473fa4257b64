"""Pins oracle_qk_norm_rope_gate (the Qwen attention producer,
native/src/inferfabric_acl.cpp:1236-1341; CPU statement
crates/inferfabric-cli/src/npu_probe/attention.rs:35-64) by properties the
mathematics fixes, each computed here independently of the oracle's code:
  * position 0 rotates nothing: the output is the bf16 norm itself, checked
    against a float64 RMS norm;
  * the rotation keeps each (j, j+32) pair's length (within bf16 rounding);
  * with gamma = 1 the normalised head has unit RMS;
  * a constant head normalises to sign(c) * gamma;
  * at position 1 the first pair of an all-ones head is (cos 1 - sin 1, cos 1 + sin 1)
    with bf16 cos/sin (float64 libm values, rounded);
  * the gate is the bf16 sigmoid: exactly 1/2 at 0, and monotone;
  * k heads use the k gamma and are unpacked (stride 256), q heads the q gamma
    and the first half of a 512-wide packed head.
"""
import numpy as np

import oracle


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_val(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rand_inputs(rng, batch):
    pq = bf16_bits(rng.standard_normal((batch, 8, 512)) * 1.3)
    k = bf16_bits(rng.standard_normal((batch, 2, 256)) * 0.7)
    qg = bf16_val(bf16_bits(rng.uniform(-0.3, 0.3, 256))) + np.float32(1)
    kg = bf16_val(bf16_bits(rng.uniform(-0.3, 0.3, 256))) + np.float32(1)
    return pq, k, qg.astype(np.float32), kg.astype(np.float32)


def norm64(x_bits, gamma):
    x = bf16_val(x_bits).astype(np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    return x * inv * gamma.astype(np.float64)


def test_position_zero_is_the_bf16_norm():
    rng = np.random.default_rng(1)
    pq, k, qg, kg = rand_inputs(rng, 4)
    q, ko, _ = oracle.qk_norm_rope_gate(pq, k, qg, kg, np.zeros(4, np.int64))
    eq = norm64(pq[..., :256], qg)
    ek = norm64(k, kg)
    for got, exp in ((q, eq), (ko, ek)):
        g = bf16_val(got).astype(np.float64)
        # one bf16 rounding of a value computed in fp32: within 2^-8 relative
        assert np.all(np.abs(g - exp) <= np.abs(exp) * 2.0 ** -8 + 1e-30)
        assert (bf16_bits(exp.astype(np.float32)) == got).mean() > 0.98


def test_rotation_keeps_pair_lengths_and_passes_the_rest():
    rng = np.random.default_rng(2)
    pq, k, qg, kg = rand_inputs(rng, 3)
    pos = np.array([1, 77, 40000], np.int64)
    q0, k0, _ = oracle.qk_norm_rope_gate(pq, k, qg, kg, np.zeros(3, np.int64))
    q, ko, _ = oracle.qk_norm_rope_gate(pq, k, qg, kg, pos)
    for rot, base in ((q, q0), (ko, k0)):
        assert np.array_equal(rot[..., 64:], base[..., 64:])
        a, b = bf16_val(base[..., :32]), bf16_val(base[..., 32:64])
        c, d = bf16_val(rot[..., :32]), bf16_val(rot[..., 32:64])
        l0 = np.sqrt(a.astype(np.float64) ** 2 + b.astype(np.float64) ** 2)
        l1 = np.sqrt(c.astype(np.float64) ** 2 + d.astype(np.float64) ** 2)
        # bf16 cos/sin (|e| <= 2^-9 each) and three roundings per component
        assert np.all(np.abs(l1 - l0) <= 0.02 * l0 + 1e-3)
        assert not np.array_equal(rot[..., :64], base[..., :64])


def test_unit_rms_constant_heads_and_gamma_routing():
    rng = np.random.default_rng(3)
    pq, k, _, _ = rand_inputs(rng, 2)
    ones = np.ones(256, np.float32)
    q, ko, _ = oracle.qk_norm_rope_gate(pq, k, ones, ones, np.zeros(2, np.int64))
    rms = np.sqrt((bf16_val(q).astype(np.float64) ** 2).mean(-1))
    assert np.all(np.abs(rms - 1) < 4e-3)
    # constant heads: c / sqrt(c^2 + 1e-6) rounds to 1 for |c| >= 1/8
    pq[:] = bf16_bits(np.float32(-0.5))
    k[:] = bf16_bits(np.float32(2.0))
    qg = np.full(256, 1.5, np.float32)
    kg = np.full(256, 0.75, np.float32)
    q, ko, _ = oracle.qk_norm_rope_gate(pq, k, qg, kg, np.zeros(2, np.int64))
    assert np.all(bf16_val(q) == -1.5)
    assert np.all(bf16_val(ko) == 0.75)


def test_hand_rotation_at_position_one():
    pq = np.full((1, 8, 512), bf16_bits(np.float32(1.0)), np.uint16)
    k = np.full((1, 2, 256), bf16_bits(np.float32(1.0)), np.uint16)
    ones = np.ones(256, np.float32)
    q, ko, _ = oracle.qk_norm_rope_gate(pq, k, ones, ones, np.array([1], np.int64))
    for j in range(32):
        f = np.float32(1.0) / np.float32(np.power(np.float64(1e7), j / 32.0))
        c = bf16_val(bf16_bits(np.float32(np.cos(np.float64(f)))))
        s = bf16_val(bf16_bits(np.float32(np.sin(np.float64(f)))))
        re = bf16_val(bf16_bits(c - s))
        im = bf16_val(bf16_bits(c + s))
        for out in (q[0, 3], ko[0, 1]):
            assert abs(bf16_val(out[j]) - re) <= abs(re) * 2 ** -7 + 1e-6, j
            assert abs(bf16_val(out[j + 32]) - im) <= abs(im) * 2 ** -7 + 1e-6, j
    assert bf16_val(q[0, 0, 0]) == bf16_val(bf16_bits(np.float32(np.cos(1.0) - np.sin(1.0))))


def test_gate_is_bf16_sigmoid():
    rng = np.random.default_rng(4)
    pq, k, qg, kg = rand_inputs(rng, 2)
    pq[0, :, 256:] = 0
    g_in = np.linspace(-12, 12, 256, dtype=np.float32)
    pq[1, :, 256:] = bf16_bits(g_in)
    _, _, gate = oracle.qk_norm_rope_gate(pq, k, qg, kg, np.zeros(2, np.int64))
    assert np.all(bf16_val(gate[0]) == 0.5)
    x = bf16_val(pq[1, 0, 256:]).astype(np.float64)
    exp = 1.0 / (1.0 + np.exp(-x))
    got = bf16_val(gate[1, 0]).astype(np.float64)
    assert np.all(np.abs(got - exp) <= exp * 2.0 ** -8)
    assert np.all(np.diff(got) >= 0)
