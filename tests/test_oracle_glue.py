"""Pins the oracle's Gemma 4 glue (orc_gelu_tanh / orc_gelu_mul,
src/cpu.rs:144-149; orc_rope_neox_in_place, src/cpu.rs:151-193) before the
GPU is checked against it: the reference's own known answers
(src/cpu.rs:798-818), float64 evaluations of the same formulas, and the
invariants the mathematics fixes (position 0 is the identity, a rotation
keeps each pair's length, pairs past rotated_pairs are untouched)."""
import numpy as np
import pytest

from oracle import capi

U = 2.0 ** -24


# ---- GELU ------------------------------------------------------------------------

def test_gelu_known_answers():
    # src/cpu.rs:798-802
    assert capi.gelu_tanh(0.0) == 0.0
    assert abs(capi.gelu_tanh(1.0) - 0.841192) < 1e-6


def gelu64(v):
    v = np.asarray(v, dtype=np.float64)
    return 0.5 * v * (1.0 + np.tanh(0.7978846 * (v + 0.044715 * v ** 3)))


def test_gelu_matches_float64_within_a_few_roundings():
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(4000) * 3, np.linspace(-12, 12, 1001)]).astype(np.float32)
    got = np.array([capi.gelu_tanh(float(x)) for x in v], dtype=np.float64)
    want = gelu64(v)
    # seven roundings and tanhf's own error, relative to the terms' sizes
    bound = 16 * U * (np.abs(v) + np.abs(want)) + 1e-30
    assert (np.abs(got - want) <= bound).all()


def test_gelu_saturates_and_mul_is_the_product():
    assert capi.gelu_tanh(60.0) == 60.0  # tanh rounds to 1
    assert capi.gelu_tanh(-60.0) == 0.0
    gate = np.array([-80.0, -51.0, 37.0, 66.0, 90.0], np.float32)
    up = np.array([2.0, -3.0, 4.0, -5.0, 6.0], np.float32)
    out = capi.gelu_mul(gate, up)
    want = np.array([np.float32(capi.gelu_tanh(float(g))) * u for g, u in zip(gate, up)], np.float32)
    assert np.array_equal(out, want)


# ---- NeoX RoPE -------------------------------------------------------------------

def test_rope_known_answer():
    # src/cpu.rs:805-817: one head of 4, one pair, position 1, theta 1
    out = capi.rope_neox([1.0, 2.0, 3.0, 4.0], 1, 4, 1, 1, 1.0)
    s, c = np.sin(1.0), np.cos(1.0)
    assert abs(out[0] - (c - 3.0 * s)) < 1e-6 and out[1] == 2.0
    assert abs(out[2] - (s + 3.0 * c)) < 1e-6 and out[3] == 4.0


def rope64(values, heads, hd, pairs, position, theta):
    v = np.array(values, dtype=np.float64).reshape(heads, hd).copy()
    half = hd // 2
    for p in range(pairs):
        exponent = np.float32(-(2.0 * p)) / np.float32(hd)  # the f32 exponent the formula rounds to
        angle = position * np.float64(theta) ** np.float64(exponent)
        a, b = v[:, p].copy(), v[:, half + p].copy()
        v[:, p] = a * np.cos(angle) - b * np.sin(angle)
        v[:, half + p] = a * np.sin(angle) + b * np.cos(angle)
    return v.ravel()


@pytest.mark.parametrize("heads,hd,pairs,position,theta", [(3, 16, 6, 37, 10000.0), (2, 256, 128, 4095, 1e6),
                                                           (4, 64, 16, 70000, 10000.0), (1, 8, 4, 1, 1.0)])
def test_rope_matches_float64_up_to_the_angle_rounding(heads, hd, pairs, position, theta):
    rng = np.random.default_rng(heads * 100 + hd)
    v = rng.standard_normal(heads * hd).astype(np.float32)
    got = capi.rope_neox(v, heads, hd, pairs, position, theta).astype(np.float64)
    want = rope64(v, heads, hd, pairs, position, theta)
    # the f32 angle is within a few ulp of position * theta^e; each output
    # moves by at most |a| + |b| times that, plus its own four roundings
    half = hd // 2
    va = np.abs(v.reshape(heads, hd)).astype(np.float64)
    mag = np.zeros((heads, hd))
    mag[:, :half] = va[:, :half] + va[:, half:]
    mag[:, half:] = mag[:, :half]
    angles = np.array([position * float(theta) ** float(np.float32(-2.0 * p) / np.float32(hd)) for p in range(half)])
    ang = np.concatenate([angles, angles])
    bound = mag * (4 * U * np.maximum(ang, 1.0) + 8 * U)
    assert (np.abs(got - want) <= bound.ravel()).all()


def test_rope_invariants():
    rng = np.random.default_rng(9)
    heads, hd, pairs = 5, 32, 10
    v = rng.standard_normal(heads * hd).astype(np.float32)
    # position 0: every angle is 0, the rotation is the identity, exactly
    assert np.array_equal(capi.rope_neox(v, heads, hd, pairs, 0, 10000.0), v)
    out = capi.rope_neox(v, heads, hd, pairs, 123, 10000.0).reshape(heads, hd).astype(np.float64)
    x = v.reshape(heads, hd).astype(np.float64)
    half = hd // 2
    # untouched dimensions: pairs p >= rotated_pairs in both halves
    assert np.array_equal(out[:, pairs:half], x[:, pairs:half])
    assert np.array_equal(out[:, half + pairs:], x[:, half + pairs:])
    # each rotated pair keeps its length
    n0 = x[:, :pairs] ** 2 + x[:, half:half + pairs] ** 2
    n1 = out[:, :pairs] ** 2 + out[:, half:half + pairs] ** 2
    assert np.all(np.abs(n1 - n0) <= 16 * U * n0 + 1e-12)


def test_rope_errors_in_the_reference_order():
    v = np.zeros(8, np.float32)
    assert capi.rope_neox_status(v, 3, 4, 1, 0, 1.0)[0] == capi.INVALID_ROPE_SHAPE
    assert capi.rope_neox_status(v, 2 ** 62, 2 ** 3, 1, 0, 1.0)[0] == capi.INVALID_ROPE_SHAPE  # overflow
    assert capi.rope_neox_status(np.zeros(6, np.float32), 2, 3, 1, 0, 1.0)[0] == capi.INVALID_ROPE_PAIRS
    assert capi.rope_neox_status(v, 2, 4, 3, 0, 1.0)[0] == capi.INVALID_ROPE_PAIRS
    assert capi.rope_neox_status(v, 2, 4, 1, 0, 0.0)[0] == capi.INVALID_POSITIVE_PARAMETER
    assert capi.rope_neox_status(v, 2, 4, 1, 0, float("nan"))[0] == capi.INVALID_POSITIVE_PARAMETER
    status, out = capi.rope_neox_status(np.ones(8, np.float32), 2, 4, 0, 5, 1.0)  # no pairs: unchanged
    assert status == capi.OK and np.array_equal(out, np.ones(8, np.float32))


def test_planted_mistake_in_the_restatement_is_caught():
    # a transposed pair (second' = first cos + second sin) would keep lengths
    # but not match float64: the float64 comparison above catches it
    heads, hd, pairs, pos = 1, 8, 4, 3
    v = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    good = capi.rope_neox(v, heads, hd, pairs, pos, 10000.0)
    bad = good.copy()
    bad[4], bad[0] = good[0], good[4]
    want = rope64(v, heads, hd, pairs, pos, 10000.0)
    assert np.abs(good - want).max() < 1e-5 and np.abs(bad - want).max() > 1e-2
