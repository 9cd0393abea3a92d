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


# ---- per-output-channel agreement -------------------------------------------
#
# rel_err divides every element's error by the largest |r| of the vector, so
# an output channel whose weights are 100x smaller than the largest is
# checked 100x less closely.  The channel measure divides each element's
# error by that element's own condition scale
#     S_i = sum_c |W_ic| |x_c|
# (float64, over the exactly dequantized weights), the quantity every
# dot-product error bound is proportional to: a relative perturbation u of
# the weights, the activations or the running sums moves y_i by at most
# about u * S_i, whatever the sizes of the other channels.  The GPU result is
# compared with the exact float64 product, and so is the oracle's
# sequential fp32 fold (printed beside it).
#
# Bars, from the error model of each path:
#  * GEMV (int8 records: 22 bits per 256-value block; fp16 hi/lo pairs: 22
#    bits per token) -- the activation rounding is at most 2^-22 of a
#    block's or token's largest |x|, under 2^-19 of S_i for Gaussian data,
#    and the fp32 partial sums add at most gamma_n S_i over n <= cols/16 + 64
#    roundings (4.6e-5 at 12288 columns): CHANNEL_TOL_GEMV = 1e-4.
#  * GEMM (one fp16 rounding per weight factor and per weight, 2^-11 each,
#    A exact above 2^-17 of its quarter's maximum): the worst case is a few
#    2^-11 of S_i, CHANNEL_TOL_GEMM = 2e-3.  The measured values sit two to
#    three orders below these bars; the tests print them.
CHANNEL_TOL_GEMV = 1e-4
CHANNEL_TOL_GEMM = 2e-3


def dense_rows(kind, rows, cols, w, first=0, count=None):
    """float64 [count][cols] dequantization of rows first.. of an encoded
    matrix (the oracle's decoders, bit-exact with the reference's)."""
    from oracle import capi  # test infrastructure only
    count = rows - first if count is None else count
    rb = w.size // rows
    part = np.ascontiguousarray(w[first * rb:(first + count) * rb])
    return capi.dequantize(kind, part, count * cols).reshape(count, cols).astype(np.float64)


def exact_products(kind, rows, cols, w, x, chunk=8192):
    """(exact, S): the float64 products W x and |W| |x| for x [cols] or
    [tokens][cols], one output row per weight row (shape [rows] or
    [tokens][rows])."""
    x = np.asarray(x, dtype=np.float64)
    xs = x.reshape(-1, cols)
    exact = np.zeros((xs.shape[0], rows))
    scale = np.zeros((xs.shape[0], rows))
    ax = np.abs(xs)
    for r0 in range(0, rows, chunk):
        n = min(chunk, rows - r0)
        d = dense_rows(kind, rows, cols, w, r0, n)
        exact[:, r0:r0 + n] = xs @ d.T
        scale[:, r0:r0 + n] = ax @ np.abs(d).T
    if x.ndim == 1:
        return exact[0], scale[0]
    return exact, scale


def channel_err(a, exact, scale) -> float:
    """max_i |a_i - exact_i| / S_i (elements with S_i = 0 must be exact)."""
    a = np.asarray(a, dtype=np.float64)
    err = np.abs(a - exact)
    zero = scale == 0
    if np.any(err[zero] != 0):
        return float("inf")
    return float((err[~zero] / scale[~zero]).max()) if np.any(~zero) else 0.0


def assert_channel_close(a, exact, scale, tol, what=""):
    e = channel_err(a, exact, scale)
    assert e <= tol, f"{what}: per-channel error {e:.3e} of S_i (bar {tol:.1e})"
    return e


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
