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
