"""Agreement measures used by the parity tests.

The north star's bar for dot products and GEMM outputs (fp32 accumulation
in a different order than the CPU's sequential fold):
  * rel_err = max_i |a_i - r_i| / max_i |r_i|  <= 1e-3
  * cosine(a, r) >= 0.99999
and, where the shape is the reference's own Metal fixture, its per-element
tolerance |a - r| <= max(5e-4, 2e-5 * |r|) (src/metal.rs:2041-2050).
Integer and index results (dequantized bits, argmax, expert ids) must be
identical.
"""
import numpy as np

REL_TOL = 1e-3
COS_TOL = 0.99999


def rel_err(a, r) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    r = np.asarray(r, dtype=np.float64).ravel()
    scale = np.abs(r).max()
    return float(np.abs(a - r).max() / scale) if scale > 0 else float(np.abs(a - r).max())


def cosine(a, r) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    r = np.asarray(r, dtype=np.float64).ravel()
    na, nr = np.linalg.norm(a), np.linalg.norm(r)
    if na == 0 and nr == 0:
        return 1.0
    return float(a @ r / (na * nr))


def assert_close(a, r, what=""):
    e, c = rel_err(a, r), cosine(a, r)
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    assert e <= REL_TOL and c >= COS_TOL, f"{what}: rel_err={e:.3e} cosine={c:.8f}"
    return e, c


def assert_metal_tolerance(a, r, what=""):
    a = np.asarray(a, dtype=np.float32)
    r = np.asarray(r, dtype=np.float32)
    tol = np.maximum(5e-4, np.abs(r) * 2e-5)
    bad = np.nonzero(np.abs(a - r) > tol)[0]
    assert bad.size == 0, f"{what}: {bad.size} elements outside max(5e-4, 2e-5|r|), first {bad[:5]}"


def top2_gap(v) -> float:
    s = np.sort(np.asarray(v, dtype=np.float64).ravel())
    return float(s[-1] - s[-2]) if s.size > 1 else float("inf")


# ---- decode attention --------------------------------------------------------
#
# Scores are the reference's sequential fp32 fma fold over the head dimension
# (src/gemma4/cpu.rs:921-927), which the GPU reproduces bit for bit; what may
# differ is exp, the order of the sums and the normalisation.  The budget
# below bounds those differences against float64 arithmetic on the same fp32
# scores, per output element, with u = 2^-24:
#   |a - exact| <= u * (F * W + 4 * W2)
#   W  = sum_j p_j |v_j|                      (every relative error of p_j and
#                                              of the running sums lands here)
#   W2 = sum_j p_j |v_j| (|s_j - M| + |s_j|)   (rounding of s_j - max before exp,
#                                              and a last-place score difference)
# F counts the rounding steps on the longest path: for the GPU's chunked
# evaluation at most 512 sequential terms per chunk, the tree and the chunk
# merge (600 + visible / 200); for the CPU fold 2 * visible + 16.
U32 = 2.0 ** -24


def fp32_fold_scores(q, k):
    """Sequential fp32 fma fold s = fma(q[d], k[:, d], s), d ascending, for one
    query row q [hd] against key rows k [n][hd]: each step adds the exact
    product in float64 and rounds to float32."""
    s = np.zeros(k.shape[0], dtype=np.float32)
    q = q.astype(np.float64)
    for d in range(k.shape[1]):
        s = (s.astype(np.float64) + q[d] * k[:, d].astype(np.float64)).astype(np.float32)
    return s


def attention_exact(query, keys, values, capacity, width, query_heads, kv_heads, head_dim, start, visible):
    """(out64, W, W2, scores) of one decode-attention step over a ring of
    `capacity` slots: float64 softmax and weighted sum of the fp32 fold
    scores, and the error weights of the budget above, all [query_heads][hd]."""
    q = np.asarray(query, dtype=np.float32).reshape(query_heads, head_dim)
    kr = np.asarray(keys, dtype=np.float32).reshape(capacity, kv_heads, head_dim)
    vr = np.asarray(values, dtype=np.float32).reshape(capacity, kv_heads, head_dim)
    slots = (start + np.arange(visible)) % capacity
    group = query_heads // kv_heads
    out = np.zeros((query_heads, head_dim))
    w = np.zeros((query_heads, head_dim))
    w2 = np.zeros((query_heads, head_dim))
    scores = np.zeros((query_heads, visible), dtype=np.float32)
    for h in range(query_heads):
        kv = h // group
        k = kr[slots, kv, :]
        v = vr[slots, kv, :].astype(np.float64)
        s = fp32_fold_scores(q[h], k)
        scores[h] = s
        s64 = s.astype(np.float64)
        m = s64.max()
        e = np.exp(s64 - m)
        p = e / e.sum()
        out[h] = p @ v
        w[h] = p @ np.abs(v)
        w2[h] = (p * (np.abs(s64 - m) + np.abs(s64))) @ np.abs(v)
    return out, w, w2, scores


def attention_budget(w, w2, visible, sequential=False):
    f = 2.0 * visible + 16 if sequential else 600.0 + visible / 200.0
    return U32 * (f * w + 4.0 * w2) + 1e-30


def assert_attention_close(a, exact, w, w2, visible, what="", sequential=False):
    a = np.asarray(a, dtype=np.float64).reshape(exact.shape)
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    budget = attention_budget(w, w2, visible, sequential)
    excess = np.abs(a - exact) / budget
    worst = float(excess.max())
    assert worst <= 1.0, f"{what}: error {worst:.3f}x the budget at {np.unravel_index(excess.argmax(), a.shape)}"
    return worst
