"""Pins the oracle's decode attention (orc_attention, src/gemma4/cpu.rs:900-946
with the ring addressing of metal/kernels.metal:486-578) before the GPU is
checked against it: the reference's own known answers, float64 arithmetic on
the same fp32 scores within a stated rounding budget, closed forms (equal
values, one dominant score) and ring-rotation invariance."""
import numpy as np
import pytest

from oracle import capi
from tests.tolerance import assert_attention_close, attention_exact, fp32_fold_scores


def run(query, keys, values, capacity, width, qh, kvh, hd, start, visible):
    return capi.attention(query, keys, values, capacity, width, qh, kvh, hd, start, visible)


# ---- the reference's known answers -------------------------------------------

def test_grouped_attention_uses_the_matching_kv_head():
    # src/gemma4/cpu.rs:967-976: 4 query heads over 2 KV heads read KV head
    # h / 2 (a mapping h % 2 would give [2, 3, 5, 7, 2, 3, 5, 7])
    out = run([1, 0, 1, 0, 0, 1, 0, 1], [1, 0, 0, 1], [2, 3, 5, 7], 1, 4, 4, 2, 2, 0, 1)
    assert out.tolist() == [2, 3, 2, 3, 5, 7, 5, 7]


def test_sliding_attention_ignores_values_outside_the_window():
    # src/gemma4/cpu.rs:978-985: two positions, window 1
    out = run([1, 0], [1, 0, 1, 0], [100, 100, 2, 4], 2, 2, 1, 1, 2, 1, 1)
    assert out.tolist() == [2, 4]


def test_resident_cache_wraps_at_the_sliding_window():
    # src/metal.rs:2543-2570: capacity 2, positions 0, 1, 2 in slots 0, 1, 0;
    # the query sees positions 1 and 2 with equal scores
    keys = [1, 0, 1, 0]
    values = [6, 8, 2, 4]  # slot 0 now holds position 2
    out = run([1, 0], keys, values, 2, 2, 1, 1, 2, 1, 2)
    assert out.tolist() == [4, 6]


def test_grouped_sliding_attention_known_case():
    # src/metal.rs:2499-2541's inputs: 4 query heads, 2 KV heads, head
    # dimension 2, three positions, window 2 (positions 1 and 2)
    query = np.array([1.0, -0.5, 0.25, 0.75, -0.5, 1.0, 0.6, -0.2], dtype=np.float32)
    keys = np.array([0.5, 0.1, -0.2, 0.8, 0.9, -0.4, 0.3, 0.7, -0.6, 0.2, 1.0, -0.5], dtype=np.float32)
    values = np.array([10.0, 20.0, 30.0, 40.0, 1.0, 2.0, 3.0, 4.0, -2.0, 0.5, 7.0, -3.0], dtype=np.float32)
    out = run(query, keys, values, 3, 4, 4, 2, 2, 1, 2)
    exact, w, w2, _ = attention_exact(query, keys, values, 3, 4, 4, 2, 2, 1, 2)
    assert_attention_close(out, exact, w, w2, 2, "grouped sliding", sequential=True)
    # the reference's own tolerance for this case
    assert np.abs(out - exact.ravel()).max() <= 2e-6


# ---- float64 on the same scores --------------------------------------------------

CASES = [
    # qh, kvh, hd, capacity, start, visible, scale
    (1, 1, 2, 7, 0, 7, 1.0),
    (4, 2, 8, 16, 5, 16, 1.0),       # ring wrap
    (3, 1, 5, 33, 40, 33, 1.0),      # group 3, odd head dimension, wrap
    (8, 2, 64, 300, 0, 257, 0.125),
    (16, 8, 256, 128, 1000, 128, 0.0625),
    (16, 2, 512, 200, 123, 200, 0.044),
    (6, 3, 16, 50, 0, 50, 3.0),      # large scores: softmax nearly one-hot
]


@pytest.mark.parametrize("qh,kvh,hd,capacity,start,visible,scale", CASES)
def test_oracle_within_the_rounding_budget_of_float64(qh, kvh, hd, capacity, start, visible, scale):
    rng = np.random.default_rng(qh * 1000 + hd + capacity)
    width = kvh * hd
    q = (rng.standard_normal(qh * hd) * scale).astype(np.float32)
    k = rng.standard_normal(capacity * width).astype(np.float32)
    v = rng.standard_normal(capacity * width).astype(np.float32)
    out = run(q, k, v, capacity, width, qh, kvh, hd, start, visible)
    exact, w, w2, _ = attention_exact(q, k, v, capacity, width, qh, kvh, hd, start, visible)
    assert_attention_close(out, exact, w, w2, visible, "oracle", sequential=True)


def test_fold_scores_are_the_sequential_fma():
    # the emulated fold against exact rational arithmetic on a few rows
    from fractions import Fraction
    rng = np.random.default_rng(5)
    q = rng.standard_normal(37).astype(np.float32)
    k = rng.standard_normal((5, 37)).astype(np.float32)
    s = fp32_fold_scores(q, k)
    for r in range(5):
        acc = np.float32(0)
        for d in range(37):
            exact = Fraction(float(q[d])) * Fraction(float(k[r, d])) + Fraction(float(acc))
            acc = np.float32(float(exact))  # one rounding of the exact value: fma
        assert acc == s[r]


# ---- closed forms and invariants -------------------------------------------------

def test_equal_values_give_that_value():
    rng = np.random.default_rng(11)
    qh, kvh, hd, n = 4, 2, 16, 40
    width = kvh * hd
    row = rng.standard_normal(width).astype(np.float32)
    v = np.tile(row, n)
    k = rng.standard_normal(n * width).astype(np.float32)
    q = rng.standard_normal(qh * hd).astype(np.float32) * 0.25
    out = run(q, k, v, n, width, qh, kvh, hd, 0, n).reshape(qh, hd)
    for h in range(qh):
        expect = row.reshape(kvh, hd)[h // 2]
        # sum_j p_j = 1 up to the n-term rounding of the sums
        assert np.allclose(out[h], expect, rtol=4 * n * 2.0 ** -24, atol=0)


def test_one_dominant_score_selects_its_value_row():
    qh, kvh, hd, n = 2, 1, 4, 9
    k = np.zeros((n, hd), dtype=np.float32)
    k[6] = [100, 0, 0, 0]  # score 100 * 100 against 0 elsewhere: exp(-1e4) is 0
    v = np.arange(n * hd, dtype=np.float32).reshape(n, hd)
    q = np.array([100, 0, 0, 0] * qh, dtype=np.float32)
    out = run(q, k.ravel(), v.ravel(), n, hd, qh, kvh, hd, 0, n).reshape(qh, hd)
    assert (out == v[6]).all()


def test_ring_rotation_leaves_the_result_bit_identical():
    rng = np.random.default_rng(3)
    qh, kvh, hd, cap = 4, 2, 8, 24
    width = kvh * hd
    seq_k = rng.standard_normal((cap, width)).astype(np.float32)
    seq_v = rng.standard_normal((cap, width)).astype(np.float32)
    q = rng.standard_normal(qh * hd).astype(np.float32)
    base = run(q, seq_k, seq_v, cap, width, qh, kvh, hd, 0, cap)
    for start in (1, 7, 23, 24, 1000):
        # position start + j lives in slot (start + j) % cap
        slots = (start + np.arange(cap)) % cap
        k = np.empty_like(seq_k)
        v = np.empty_like(seq_v)
        k[slots] = seq_k
        v[slots] = seq_v
        out = run(q, k, v, cap, width, qh, kvh, hd, start, cap)
        assert np.array_equal(out.view(np.uint32), base.view(np.uint32)), start


def test_statuses():
    q = np.ones(2, dtype=np.float32)
    k = np.ones(4, dtype=np.float32)
    status, _ = capi.attention_status(q, k, k, 2, 2, 1, 1, 2, 0, 0)
    assert status == capi.EMPTY_INPUT
    status, _ = capi.attention_status([np.nan, 0], k, k, 2, 2, 1, 1, 2, 0, 2)
    assert status == capi.NON_FINITE
    status, _ = capi.attention_status([np.inf, 0], k, k, 2, 2, 1, 1, 2, 0, 2)
    assert status == capi.NON_FINITE  # +inf scores
    status, _ = capi.attention_status([-np.inf, 0], k, k, 2, 2, 1, 1, 2, 0, 2)
    assert status == capi.NON_FINITE  # every score -inf
    kk = np.array([1, 0, -1, 0], dtype=np.float32)
    status, out = capi.attention_status([-np.inf, 0], kk, kk, 2, 2, 1, 1, 2, 0, 2)
    assert status == capi.NON_FINITE  # scores -inf and +inf: the +inf one
