"""ctypes binding of ``libdm_oracle.so`` (the C restatement of ``src/cpu.rs``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libdm_oracle.so")

# CpuError codes, src/cpu.rs:10-96 (mirrors dm_oracle.h)
OK = 0
UNSUPPORTED_TYPE = 1
INVALID_ELEMENT_COUNT = 2
INVALID_BYTE_LENGTH = 3
OVERFLOW = 4
INVALID_INPUT_LENGTH = 5
INVALID_OUTPUT_LENGTH = 6
EMPTY_INPUT = 7
INVALID_VECTOR_LENGTH = 8
NON_FINITE = 9
INVALID_TOP_K = 10
INVALID_POSITIVE_PARAMETER = 11
INVALID_LAYER = 12
INVALID_EXPERT = 13
ALL_SLOTS_PINNED = 14
NO_SLOTS = 15
INVALID_ROPE_SHAPE = 16
INVALID_ROPE_PAIRS = 17


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: oracle status {code}")
        self.code = code


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off); always
    rebuilds, so a changed compiler or flag cannot leave a stale library."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_szp = ctypes.POINTER(ctypes.c_size_t)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_sz = ctypes.c_size_t


def _declare(l: ctypes.CDLL) -> None:
    l.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    l.orc_f16_to_f32.restype = ctypes.c_float
    l.orc_row_byte_len.argtypes = [ctypes.c_uint32, ctypes.c_uint64, _u64p]
    l.orc_scale_min_q4_k.argtypes = [_sz, _u8p, _u8p, _u8p]
    l.orc_scale_min_q4_k.restype = None
    l.orc_dequantize.argtypes = [ctypes.c_uint32, _u8p, _sz, _f32p, _sz]
    l.orc_matvec.argtypes = [ctypes.c_uint32, _sz, _sz, _u8p, _sz, _f32p, _sz, _f32p, _sz, ctypes.c_int]
    l.orc_matvec_bf16.argtypes = [_sz, _sz, _u16p, _f32p, _f32p, ctypes.c_int]
    l.orc_argmax.argtypes = [_f32p, _sz, _szp]
    l.orc_softmax_in_place.argtypes = [_f32p, _sz]
    l.orc_top_k_softmax.argtypes = [_f32p, _sz, _sz, _szp, _f32p]
    l.orc_rms_norm.argtypes = [_f32p, _sz, _f32p, _sz, ctypes.c_float, _f32p, _sz]
    l.orc_silu.argtypes = [ctypes.c_float]
    l.orc_softcap_in_place.argtypes = [_f32p, _sz, ctypes.c_float]
    l.orc_gelu_tanh.argtypes = [ctypes.c_float]
    l.orc_gelu_tanh.restype = ctypes.c_float
    l.orc_gelu_mul.argtypes = [_f32p, _f32p, _sz, _f32p]
    l.orc_gelu_mul.restype = None
    l.orc_rope_neox_in_place.argtypes = [_f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_float]
    l.orc_softcap_in_place.restype = ctypes.c_int
    l.orc_silu.restype = ctypes.c_float
    l.orc_silu_mul_glm.argtypes = [_f32p, _f32p, _sz, _f32p]
    l.orc_silu_mul_glm.restype = None
    l.orc_dense_ffn.argtypes = [_sz, _sz, _sz, ctypes.c_uint32, _u8p, ctypes.c_uint32, _u8p,
                                ctypes.c_uint32, _u8p, _f32p, ctypes.c_float, _f32p, ctypes.c_int]
    l.orc_moe_layer.argtypes = [_sz, _sz, _sz, _sz, _sz, _u16p, ctypes.c_uint32, _u8p,
                                ctypes.c_uint32, _u8p, _f32p, _szp, _f32p, _f32p, ctypes.c_int]
    l.orc_gemm_tokenwise.argtypes = [ctypes.c_uint32, _sz, _sz, _sz, _u16p, _u8p, _f32p, ctypes.c_int]
    l.orc_attention.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f32p]
    l.orc_st_decode_f8_e4m3fn.argtypes = [ctypes.c_uint8, _f32p]
    l.orc_st_u8_encoding.argtypes = [_sz, _sz, _sz, _sz, ctypes.POINTER(ctypes.c_int), _szp, _szp, _szp, _szp,
                                     ctypes.POINTER(ctypes.c_int)]
    l.orc_st_matvec.argtypes = [ctypes.c_int, _sz, _sz, _u8p, _f32p, _sz, _f32p, _f32p]
    l.orc_st_dequantize_row.argtypes = [ctypes.c_int, _sz, _sz, _u8p, _f32p, _sz, _sz, _f32p]
    l.orc_lru_new.argtypes = [_sz, _szp, _sz, ctypes.c_uint64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p)]
    l.orc_lru_free.argtypes = [ctypes.c_void_p]
    l.orc_lru_free.restype = None
    l.orc_lru_acquire.argtypes = [ctypes.c_void_p, _sz, _sz, _szp, ctypes.POINTER(ctypes.c_int),
                                  ctypes.POINTER(ctypes.c_int), _szp]
    l.orc_lru_set_pinned.argtypes = [ctypes.c_void_p, _sz, _sz, ctypes.c_int]
    l.orc_lru_set_pinned.restype = None
    l.orc_lru_stats.argtypes = [ctypes.c_void_p] + [_u64p] * 6
    l.orc_lru_stats.restype = None


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _check(code: int, what: str) -> None:
    if code != OK:
        raise OracleError(code, what)


def threads_default() -> int:
    return min(16, os.cpu_count() or 1)


def f16_to_f32(bits: int) -> np.float32:
    return np.float32(lib().orc_f16_to_f32(bits))


def row_byte_len(ggml_type: int, elements: int) -> int:
    out = ctypes.c_uint64()
    _check(lib().orc_row_byte_len(ggml_type, elements, ctypes.byref(out)), "row_byte_len")
    return out.value


def scale_min_q4_k(index: int, scales) -> tuple[int, int]:
    s = _c(scales, np.uint8)
    a, b = ctypes.c_uint8(), ctypes.c_uint8()
    lib().orc_scale_min_q4_k(index, _p(s, _u8p), ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def dequantize(ggml_type: int, encoded, elements: int) -> np.ndarray:
    enc = _c(encoded, np.uint8)
    out = np.zeros(elements, dtype=np.float32)
    _check(lib().orc_dequantize(ggml_type, _p(enc, _u8p), enc.size, _p(out, _f32p), elements),
           "dequantize")
    return out


def dequantize_status(ggml_type: int, encoded, elements: int) -> int:
    enc = _c(encoded, np.uint8)
    out = np.zeros(max(elements, 1), dtype=np.float32)
    return lib().orc_dequantize(ggml_type, _p(enc, _u8p), enc.size, _p(out, _f32p), elements)


def matvec(ggml_type: int, rows: int, columns: int, encoded, x, threads: int | None = None) -> np.ndarray:
    enc = _c(encoded, np.uint8)
    xin = _c(x, np.float32)
    out = np.zeros(rows, dtype=np.float32)
    _check(lib().orc_matvec(ggml_type, rows, columns, _p(enc, _u8p), enc.size, _p(xin, _f32p),
                            xin.size, _p(out, _f32p), rows, threads or threads_default()), "matvec")
    return out


def matvec_status(ggml_type: int, rows: int, columns: int, encoded, x, out_len: int) -> int:
    enc = _c(encoded, np.uint8)
    xin = _c(x, np.float32)
    out = np.zeros(max(out_len, 1), dtype=np.float32)
    return lib().orc_matvec(ggml_type, rows, columns, _p(enc, _u8p), enc.size, _p(xin, _f32p),
                            xin.size, _p(out, _f32p), out_len, 1)


def matvec_bf16(rows: int, columns: int, weights_bits, x, threads: int | None = None) -> np.ndarray:
    w = _c(weights_bits, np.uint16)
    xin = _c(x, np.float32)
    out = np.zeros(rows, dtype=np.float32)
    _check(lib().orc_matvec_bf16(rows, columns, _p(w, _u16p), _p(xin, _f32p), _p(out, _f32p),
                                 threads or threads_default()), "matvec_bf16")
    return out


def argmax(values) -> int:
    v = _c(values, np.float32)
    idx = ctypes.c_size_t()
    _check(lib().orc_argmax(_p(v, _f32p), v.size, ctypes.byref(idx)), "argmax")
    return idx.value


def argmax_status(values) -> int:
    v = _c(values, np.float32)
    idx = ctypes.c_size_t()
    return lib().orc_argmax(_p(v, _f32p) if v.size else None, v.size, ctypes.byref(idx))


def softmax(values) -> np.ndarray:
    v = np.array(values, dtype=np.float32)
    _check(lib().orc_softmax_in_place(_p(v, _f32p), v.size), "softmax")
    return v


def top_k_softmax(logits, k: int) -> list[tuple[int, float]]:
    v = _c(logits, np.float32)
    ids = np.zeros(max(k, 1), dtype=np.uintp)
    probs = np.zeros(max(k, 1), dtype=np.float32)
    _check(lib().orc_top_k_softmax(_p(v, _f32p), v.size, k, ids.ctypes.data_as(_szp),
                                   _p(probs, _f32p)), "top_k_softmax")
    return [(int(ids[i]), float(probs[i])) for i in range(k)]


def top_k_softmax_status(logits, k: int) -> int:
    v = _c(logits, np.float32)
    ids = np.zeros(max(k, 1), dtype=np.uintp)
    probs = np.zeros(max(k, 1), dtype=np.float32)
    return lib().orc_top_k_softmax(_p(v, _f32p), v.size, k, ids.ctypes.data_as(_szp), _p(probs, _f32p))


def rms_norm(x, weight=None, epsilon: float = 1e-6) -> np.ndarray:
    v = _c(x, np.float32)
    out = np.zeros_like(v)
    w = None if weight is None else _c(weight, np.float32)
    _check(lib().orc_rms_norm(_p(v, _f32p), v.size, None if w is None else _p(w, _f32p),
                              0 if w is None else w.size, epsilon, _p(out, _f32p), out.size), "rms_norm")
    return out


def rms_norm_status(x, weight, epsilon: float, out_len: int) -> int:
    v = _c(x, np.float32)
    out = np.zeros(max(out_len, 1), dtype=np.float32)
    w = None if weight is None else _c(weight, np.float32)
    return lib().orc_rms_norm(_p(v, _f32p) if v.size else None, v.size,
                              None if w is None else _p(w, _f32p), 0 if w is None else w.size,
                              epsilon, _p(out, _f32p), out_len)


def silu(value: float) -> np.float32:
    return np.float32(lib().orc_silu(value))


def softcap(values, cap: float) -> np.ndarray:
    out = np.array(values, dtype=np.float32, copy=True).ravel()
    _check(lib().orc_softcap_in_place(_p(out, _f32p), out.size, cap), "softcap")
    return out


def softcap_status(values, cap: float) -> int:
    out = np.array(values, dtype=np.float32, copy=True).ravel()
    return lib().orc_softcap_in_place(_p(out, _f32p), out.size, cap)


def gelu_tanh(value: float) -> float:
    return float(np.float32(lib().orc_gelu_tanh(value)))


def gelu_mul(gate, up) -> np.ndarray:
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.zeros_like(g)
    lib().orc_gelu_mul(_p(g, _f32p), _p(u, _f32p), g.size, _p(out, _f32p))
    return out


def rope_neox_status(values, heads: int, head_dimension: int, rotated_pairs: int, position: int,
                     theta: float) -> tuple[int, np.ndarray]:
    v = np.array(values, dtype=np.float32, copy=True).ravel()
    status = lib().orc_rope_neox_in_place(_p(v, _f32p), v.size, heads, head_dimension, rotated_pairs, position,
                                          theta)
    return status, v


def rope_neox(values, heads: int, head_dimension: int, rotated_pairs: int, position: int,
              theta: float) -> np.ndarray:
    status, v = rope_neox_status(values, heads, head_dimension, rotated_pairs, position, theta)
    _check(status, "rope_neox")
    return v


def silu_mul_glm(gate, up) -> np.ndarray:
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.zeros_like(g)
    lib().orc_silu_mul_glm(_p(g, _f32p), _p(u, _f32p), g.size, _p(out, _f32p))
    return out


def dense_ffn(batch, hidden, ffn, gate_type, gate, up_type, up, down_type, down, h,
              epsilon=1e-6, threads=None) -> np.ndarray:
    g, u, d = (_c(a, np.uint8) for a in (gate, up, down))
    hin = _c(h, np.float32)
    out = np.zeros((batch, hidden), dtype=np.float32)
    _check(lib().orc_dense_ffn(batch, hidden, ffn, gate_type, _p(g, _u8p), up_type, _p(u, _u8p),
                               down_type, _p(d, _u8p), _p(hin, _f32p), epsilon, _p(out, _f32p),
                               threads or threads_default()), "dense_ffn")
    return out


def moe_layer(batch, hidden, width, experts, k, router_bits, gu_type, gate_up_all, dn_type,
              down_all, tokens, threads=None):
    r = _c(router_bits, np.uint16)
    gu = _c(gate_up_all, np.uint8)
    dn = _c(down_all, np.uint8)
    x = _c(tokens, np.float32)
    sel = np.zeros((batch, k), dtype=np.uintp)
    wts = np.zeros((batch, k), dtype=np.float32)
    out = np.zeros((batch, hidden), dtype=np.float32)
    _check(lib().orc_moe_layer(batch, hidden, width, experts, k, _p(r, _u16p), gu_type, _p(gu, _u8p),
                               dn_type, _p(dn, _u8p), _p(x, _f32p), sel.ctypes.data_as(_szp),
                               _p(wts, _f32p), _p(out, _f32p), threads or threads_default()), "moe_layer")
    return sel.astype(np.int64), wts, out


def gemm_tokenwise(ggml_type, m, n, k, a_bits, encoded, threads=None) -> np.ndarray:
    a = _c(a_bits, np.uint16)
    enc = _c(encoded, np.uint8)
    out = np.zeros((m, n), dtype=np.float32)
    _check(lib().orc_gemm_tokenwise(ggml_type, m, n, k, _p(a, _u16p), _p(enc, _u8p), _p(out, _f32p),
                                    threads or threads_default()), "gemm_tokenwise")
    return out


ST_BF16, ST_F8_E4M3, ST_INT8_ROW, ST_INT4_GROUPED = 0, 1, 2, 3


def st_decode_f8(bits: int):
    """decode_f8_e4m3fn: the value, or None for the NaN patterns."""
    v = ctypes.c_float()
    return v.value if lib().orc_st_decode_f8_e4m3fn(bits, ctypes.byref(v)) == OK else None


def st_u8_encoding(rows: int, columns: int, encoded_len: int, scale_len: int) -> dict:
    """u8_matrix_encoding: {"format", "group_size", "scale_columns"} or
    {"error": status, "expected", "actual", "scales"}."""
    g, sc, e, a = (ctypes.c_size_t() for _ in range(4))
    fmt, bad = ctypes.c_int(), ctypes.c_int()
    r = lib().orc_st_u8_encoding(rows, columns, encoded_len, scale_len, ctypes.byref(fmt), ctypes.byref(g),
                                 ctypes.byref(sc), ctypes.byref(e), ctypes.byref(a), ctypes.byref(bad))
    if r == OK:
        return {"format": fmt.value, "group_size": g.value, "scale_columns": sc.value}
    return {"error": r, "expected": e.value, "actual": a.value, "scales": bool(bad.value)}


def st_matvec(fmt: int, rows: int, columns: int, encoded, scales, input, group_size: int = 0) -> np.ndarray:
    enc = _c(encoded, np.uint8)
    sc = _c(scales if scales is not None else np.zeros(1), np.float32)
    x = _c(input, np.float32)
    out = np.zeros(max(rows, 1), dtype=np.float32)
    _check(lib().orc_st_matvec(fmt, rows, columns, _p(enc, _u8p), _p(sc, _f32p), group_size, _p(x, _f32p),
                               _p(out, _f32p)), "st_matvec")
    return out[:rows]


def st_dequantize_row(fmt: int, rows: int, columns: int, encoded, scales, row: int, group_size: int = 0):
    enc = _c(encoded, np.uint8)
    sc = _c(scales if scales is not None else np.zeros(1), np.float32)
    out = np.zeros(max(columns, 1), dtype=np.float32)
    _check(lib().orc_st_dequantize_row(fmt, rows, columns, _p(enc, _u8p), _p(sc, _f32p), group_size, row,
                                       _p(out, _f32p)), "st_dequantize_row")
    return out[:columns]


def attention_status(query, keys, values, capacity: int, width: int, query_heads: int, kv_heads: int,
                     head_dimension: int, start: int, visible: int):
    """(status, output) of one decode-attention step over a KV ring of
    `capacity` slots of `width` floats (src/gemma4/cpu.rs:900-946)."""
    q = _c(query, np.float32).ravel()
    k = _c(keys, np.float32).ravel()
    v = _c(values, np.float32).ravel()
    assert q.size == query_heads * head_dimension and width == kv_heads * head_dimension
    assert k.size == v.size == capacity * width and visible <= capacity
    out = np.zeros(query_heads * head_dimension, dtype=np.float32)
    status = lib().orc_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), capacity, width, query_heads,
                                 kv_heads, head_dimension, start, visible, _p(out, _f32p))
    return status, out


def attention(query, keys, values, capacity: int, width: int, query_heads: int, kv_heads: int,
              head_dimension: int, start: int, visible: int) -> np.ndarray:
    status, out = attention_status(query, keys, values, capacity, width, query_heads, kv_heads,
                                   head_dimension, start, visible)
    _check(status, "attention")
    return out


class Lru:
    """src/expert.rs:44-229 slot bookkeeping (no byte movement)."""

    def __init__(self, expert_counts, slots_per_layer, gate_up_bytes, down_bytes):
        counts = np.array(expert_counts, dtype=np.uintp)
        h = ctypes.c_void_p()
        _check(lib().orc_lru_new(counts.size, counts.ctypes.data_as(_szp), slots_per_layer,
                                 gate_up_bytes, down_bytes, ctypes.byref(h)), "lru_new")
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_lru_free(self._h)
            self._h = None

    def acquire(self, layer, expert):
        slot = ctypes.c_size_t()
        hit = ctypes.c_int()
        ev = ctypes.c_int()
        eve = ctypes.c_size_t()
        _check(lib().orc_lru_acquire(self._h, layer, expert, ctypes.byref(slot), ctypes.byref(hit),
                                     ctypes.byref(ev), ctypes.byref(eve)), "lru_acquire")
        return slot.value, bool(hit.value), (eve.value if ev.value else None)

    def set_pinned(self, layer, slot, pinned):
        lib().orc_lru_set_pinned(self._h, layer, slot, int(pinned))

    def stats(self) -> dict:
        vals = [ctypes.c_uint64() for _ in range(6)]
        lib().orc_lru_stats(self._h, *[ctypes.byref(v) for v in vals])
        keys = ["hits", "misses", "evictions", "reads", "bytes_read", "resident_bytes"]
        return {k: v.value for k, v in zip(keys, vals)}
