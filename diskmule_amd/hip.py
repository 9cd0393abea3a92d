"""ctypes binding of ``libdmhip.so`` (the C ABI in ``include/dmhip.h``).

Method names, argument meaning and errors mirror the reference's Metal
backend (``src/metal.rs``: ``MetalContext``, ``MetalOwnedBuffer``,
``MetalMappedBuffer``) and expert residency (``src/expert.rs``), so callers
and tests read like the reference's own.  Errors raise :class:`HipError`
whose ``variant`` is the ``MetalError`` / ``ExpertCacheError`` variant name.
"""
from __future__ import annotations

import ctypes
import os
import weakref
from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "libdmhip.so")

# dmhip_status -> reference error variant
VARIANTS = {
    0: "Ok", 1: "NoDevice", 2: "BufferAllocation", 3: "VectorLength", 4: "VectorTooLarge",
    5: "EmptyInput", 6: "InvalidVectorLength", 7: "InvalidPositiveParameter", 8: "NonFinite",
    9: "UnsupportedTensorType", 10: "InvalidElementCount", 11: "InvalidByteLength",
    12: "Overflow", 13: "InvalidInputLength", 14: "InvalidOutputLength", 15: "InvalidTopK",
    16: "MappedRange", 17: "Command", 18: "NoSlots", 19: "InvalidLayer", 20: "InvalidExpert",
    21: "AllSlotsPinned", 22: "Cancelled", 23: "InvalidLayout", 24: "InvalidArgument", 25: "Io",
    26: "InvalidAttentionShape", 27: "KvPosition", 28: "KvWidth", 29: "KvContext",
    30: "InvalidRopeShape", 31: "InvalidRopePairs",
}

# Every function include/dmhip.h declares (checked against the header by tests).
EXPORTED_SYMBOLS = [
    "dmhip_last_error", "dmhip_last_error_detail", "dmhip_context_new", "dmhip_context_free", "dmhip_device_name",
    "dmhip_synchronize", "dmhip_stream", "dmhip_map_read_only", "dmhip_new_owned_buffer",
    "dmhip_buffer_free", "dmhip_buffer_len", "dmhip_buffer_device_ptr", "dmhip_buffer_write",
    "dmhip_buffer_read", "dmhip_copy_to_host", "dmhip_copy_to_device", "dmhip_host_alloc_pinned", "dmhip_host_free_pinned", "dmhip_rms_norm",
    "dmhip_silu_mul", "dmhip_softcap", "dmhip_argmax", "dmhip_top_k_softmax", "dmhip_matvec",
    "dmhip_matvec_mapped", "dmhip_matvec_owned", "dmhip_dequantize", "dmhip_matvec_device",
    "dmhip_matvec_batch_device", "dmhip_matvec_argmax_device", "dmhip_argmax_result", "dmhip_rms_norm_device",
    "dmhip_silu_mul_device", "dmhip_softcap_device", "dmhip_ffn_workspace_bytes", "dmhip_ffn_device",
    "dmhip_ffn_noalloc_scratch_bytes", "dmhip_ffn_device_noalloc",
    "dmhip_router_top_k_device", "dmhip_router_result", "dmhip_gemm_workspace_bytes", "dmhip_gemm_device",
    "dmhip_event_record", "dmhip_event_elapsed_ms", "dmhip_event_free",
    "dmhip_copy_device",
    "dmhip_expert_cache_new", "dmhip_expert_cache_new_file", "dmhip_expert_cache_free",
    "dmhip_expert_cache_stats_get",
    "dmhip_expert_cache_slots_per_layer", "dmhip_expert_acquire", "dmhip_expert_release",
    "dmhip_moe_layer",
    "dmhip_new_kv_layer", "dmhip_kv_layer_free", "dmhip_kv_layer_position", "dmhip_kv_layer_capacity",
    "dmhip_kv_layer_allocated_bytes", "dmhip_kv_layer_clear", "dmhip_kv_layer_truncate",
    "dmhip_kv_layer_width", "dmhip_kv_layer_keys", "dmhip_kv_layer_values", "dmhip_append_kv",
    "dmhip_append_kv_device", "dmhip_attention_cached", "dmhip_attention_cached_device",
    "dmhip_attention_result", "dmhip_attention",
    "dmhip_matvec_safetensor_mapped", "dmhip_matvec_safetensor", "dmhip_matvec_safetensor_device",
    "dmhip_add", "dmhip_gelu_mul", "dmhip_softmax", "dmhip_rope_neox_in_place", "dmhip_add_device",
    "dmhip_gelu_mul_device", "dmhip_rope_neox_device",
]

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 6, 8, 12, 14, 30

# SafeDtype (src/safetensors.rs:171-187) ids of the safetensors entry points
SAFE = {"BOOL": 0, "U8": 1, "I8": 2, "U16": 3, "I16": 4, "F16": 5, "BF16": 6, "U32": 7, "I32": 8, "F32": 9,
        "U64": 10, "I64": 11, "F64": 12, "F8_E4M3": 13, "F8_E5M2": 14}


class HipError(RuntimeError):
    """A failed call: `variant` names the MetalError / ExpertCacheError variant
    and `detail` holds that variant's fields (dmhip_last_error_detail)."""

    def __init__(self, code: int, message: str, detail: dict | None = None):
        self.code = code
        self.variant = VARIANTS.get(code, f"Unknown({code})")
        self.detail = detail or {}
        super().__init__(f"{self.variant}: {message}")


def library_path() -> str:
    return _LIB


_lib = None

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_szp = ctypes.POINTER(ctypes.c_size_t)


class _Layout(ctypes.Structure):
    _fields_ = [("expert_count", _sz), ("gate_up_offset", ctypes.c_uint64),
                ("gate_up_bytes", _sz), ("down_offset", ctypes.c_uint64), ("down_bytes", _sz)]


class _Detail(ctypes.Structure):
    _fields_ = [("status", ctypes.c_int32), ("os_error", ctypes.c_int32), ("operation", ctypes.c_char_p),
                ("argument", ctypes.c_char_p), ("kind", ctypes.c_char_p)] + \
               [(n, ctypes.c_uint64) for n in ("expected", "actual", "offset", "end", "length", "left", "right",
                                               "output", "elements", "block_elements", "k", "bytes", "layer",
                                               "expert", "count", "position", "limit")] + \
               [("reason", ctypes.c_char_p), ("heads", ctypes.c_uint64), ("head_dimension", ctypes.c_uint64)]

    # the fields each variant carries (include/dmhip.h)
    FIELDS = {
        2: ("bytes",), 3: ("left", "right", "output"), 5: ("operation",),
        6: ("operation", "argument", "expected", "actual"), 7: ("operation",), 8: ("operation",), 9: ("kind",),
        10: ("kind", "elements", "block_elements"), 11: ("kind", "expected", "actual"), 13: ("expected", "actual"),
        14: ("expected", "actual"), 15: ("k", "length"), 16: ("offset", "end", "length"), 19: ("layer", "count"),
        20: ("layer", "expert", "count"), 21: ("layer",), 25: ("os_error",), 26: ("reason",),
        27: ("expected", "actual"), 28: ("expected", "actual"), 29: ("position", "limit"),
        30: ("length", "heads", "head_dimension"),
    }

    def as_dict(self) -> dict:
        out = {}
        for name in self.FIELDS.get(self.status, ()):
            v = getattr(self, name)
            out[name] = v.decode() if isinstance(v, bytes) else v
        return out


class _Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in
                ("hits", "misses", "evictions", "reads", "bytes_read", "io_wait_ns", "resident_bytes")]


def load_library() -> ctypes.CDLL:
    """Load ``libdmhip.so``; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB):
        raise HipError(1, f"{_LIB} is missing: build it with diskmule_amd/build.py "
                          "(there is no CPU fallback)")
    lib = ctypes.CDLL(_LIB)
    sig = {
        "dmhip_last_error": ([], ctypes.c_char_p),
        "dmhip_last_error_detail": ([ctypes.POINTER(_Detail)], ctypes.c_int),
        "dmhip_context_new": ([ctypes.c_int, ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_context_free": ([_vp], None),
        "dmhip_device_name": ([_vp, ctypes.c_char_p, _sz], ctypes.c_int),
        "dmhip_synchronize": ([_vp], ctypes.c_int),
        "dmhip_stream": ([_vp], _vp),
        "dmhip_map_read_only": ([_vp, _vp, _sz, ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_new_owned_buffer": ([_vp, _sz, ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_buffer_free": ([_vp], None),
        "dmhip_buffer_len": ([_vp], _sz),
        "dmhip_buffer_device_ptr": ([_vp], _vp),
        "dmhip_buffer_write": ([_vp, _vp, _sz, _vp, _sz], ctypes.c_int),
        "dmhip_buffer_read": ([_vp, _vp, _sz, _vp, _sz], ctypes.c_int),
        "dmhip_copy_to_host": ([_vp, _vp, _vp, _sz], ctypes.c_int),
        "dmhip_copy_to_device": ([_vp, _vp, _vp, _sz], ctypes.c_int),
        "dmhip_host_alloc_pinned": ([_sz, ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_host_free_pinned": ([_vp], None),
        "dmhip_rms_norm": ([_vp, _f32p, _sz, _f32p, _sz, ctypes.c_float, _f32p, _sz], ctypes.c_int),
        "dmhip_silu_mul": ([_vp, _f32p, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_softcap": ([_vp, _f32p, _sz, ctypes.c_float, _f32p, _sz], ctypes.c_int),
        "dmhip_add": ([_vp, _f32p, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_gelu_mul": ([_vp, _f32p, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_softmax": ([_vp, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_rope_neox_in_place": ([_vp, _f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_float], ctypes.c_int),
        "dmhip_argmax": ([_vp, _f32p, _sz, _szp], ctypes.c_int),
        "dmhip_top_k_softmax": ([_vp, _f32p, _sz, _sz, _szp, _f32p], ctypes.c_int),
        "dmhip_matvec": ([_vp, _u32, _sz, _sz, _u8p, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_matvec_mapped": ([_vp, _u32, _sz, _sz, _vp, _sz, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_matvec_owned": ([_vp, _u32, _sz, _sz, _vp, _sz, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_dequantize": ([_vp, _u32, _vp, _sz, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_matvec_device": ([_vp, _u32, _sz, _sz, _vp, _sz, _vp, _vp], ctypes.c_int),
        "dmhip_matvec_batch_device": ([_vp, _u32, _sz, _sz, _sz, ctypes.POINTER(_vp), _vp, _sz, _vp, _sz],
                                      ctypes.c_int),
        "dmhip_matvec_argmax_device": ([_vp, _u32, _sz, _sz, _vp, _vp, _vp, _vp], ctypes.c_int),
        "dmhip_argmax_result": ([_vp, _szp], ctypes.c_int),
        "dmhip_rms_norm_device": ([_vp, _sz, _sz, _vp, _vp, ctypes.c_float, _vp], ctypes.c_int),
        "dmhip_silu_mul_device": ([_vp, _sz, _vp, _vp, _vp], ctypes.c_int),
        "dmhip_softcap_device": ([_vp, _sz, _vp, ctypes.c_float, _vp], ctypes.c_int),
        "dmhip_add_device": ([_vp, _sz, _vp, _vp, _vp], ctypes.c_int),
        "dmhip_gelu_mul_device": ([_vp, _sz, _vp, _vp, _vp], ctypes.c_int),
        "dmhip_rope_neox_device": ([_vp, _vp, _sz, _sz, _sz, _sz, _sz, ctypes.c_float], ctypes.c_int),
        "dmhip_ffn_workspace_bytes": ([_sz, _sz, _sz], _sz),
        "dmhip_ffn_device": ([_vp, _sz, _sz, _sz, _u32, _vp, _u32, _vp, _u32, _vp, ctypes.c_float,
                              _vp, _vp, _vp, _sz], ctypes.c_int),
        "dmhip_ffn_noalloc_scratch_bytes": ([], _sz),
        "dmhip_ffn_device_noalloc": ([_vp, _sz, _sz, _sz, _u32, _vp, _u32, _vp, _u32, _vp, ctypes.c_float,
                                      _vp, _vp], ctypes.c_int),
        "dmhip_router_top_k_device": ([_vp, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
        "dmhip_router_result": ([_vp], ctypes.c_int),
        "dmhip_gemm_workspace_bytes": ([_sz, _sz], _sz),
        "dmhip_gemm_device": ([_vp, _u32, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _sz], ctypes.c_int),
        "dmhip_event_record": ([_vp, ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_event_elapsed_ms": ([_vp, _vp, ctypes.POINTER(ctypes.c_float)], ctypes.c_int),
        "dmhip_event_free": ([_vp], None),
        "dmhip_copy_device": ([_vp, _vp, _vp, _sz], ctypes.c_int),
        "dmhip_expert_cache_new": ([_vp, _vp, _sz, ctypes.POINTER(_Layout), _sz, _sz, ctypes.POINTER(_vp)],
                                   ctypes.c_int),
        "dmhip_expert_cache_new_file": ([_vp, ctypes.c_int, ctypes.POINTER(_Layout), _sz, _sz,
                                         ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_expert_cache_free": ([_vp], None),
        "dmhip_expert_cache_stats_get": ([_vp, ctypes.POINTER(_Stats)], ctypes.c_int),
        "dmhip_expert_cache_slots_per_layer": ([_vp], _sz),
        "dmhip_expert_acquire": ([_vp, _sz, _sz, ctypes.POINTER(ctypes.c_int), _szp,
                                  ctypes.POINTER(_vp), ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_expert_release": ([_vp, _sz, _sz], ctypes.c_int),
        "dmhip_moe_layer": ([_vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _u32, _u32, _vp, _vp,
                             ctypes.POINTER(ctypes.c_uint32), _f32p], ctypes.c_int),
        "dmhip_new_kv_layer": ([_vp, _sz, _sz, ctypes.c_int, _sz, ctypes.POINTER(_vp)], ctypes.c_int),
        "dmhip_kv_layer_free": ([_vp], None),
        "dmhip_kv_layer_position": ([_vp], _sz),
        "dmhip_kv_layer_capacity": ([_vp], _sz),
        "dmhip_kv_layer_allocated_bytes": ([_vp], _sz),
        "dmhip_kv_layer_clear": ([_vp], None),
        "dmhip_kv_layer_truncate": ([_vp, _sz], None),
        "dmhip_kv_layer_width": ([_vp], _sz),
        "dmhip_kv_layer_keys": ([_vp], _vp),
        "dmhip_kv_layer_values": ([_vp], _vp),
        "dmhip_append_kv": ([_vp, _vp, _sz, _f32p, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_append_kv_device": ([_vp, _vp, _sz, _vp, _sz, _vp, _sz], ctypes.c_int),
        "dmhip_attention_cached": ([_vp, _f32p, _sz, _vp, _sz, _sz, _sz, _f32p, _sz], ctypes.c_int),
        "dmhip_attention_cached_device": ([_vp, _vp, _sz, _vp, _sz, _sz, _sz, _vp, _sz], ctypes.c_int),
        "dmhip_attention_result": ([_vp], ctypes.c_int),
        "dmhip_attention": ([_vp, _f32p, _sz, _f32p, _sz, _f32p, _sz, _sz, _sz, _sz, ctypes.c_int, _sz,
                             _f32p, _sz], ctypes.c_int),
        "dmhip_matvec_safetensor_mapped": ([_vp, _u32, _sz, _sz, _vp, _sz, _sz, _vp, _sz, _sz, _f32p, _sz, _f32p,
                                            _sz], ctypes.c_int),
        "dmhip_matvec_safetensor": ([_vp, _u32, _sz, _sz, _u8p, _sz, _f32p, _sz, _f32p, _sz, _f32p, _sz],
                                    ctypes.c_int),
        "dmhip_matvec_safetensor_device": ([_vp, _u32, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _vp], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _check(code: int) -> None:
    if code != 0:
        lib = load_library()
        msg = lib.dmhip_last_error()
        d = _Detail()
        lib.dmhip_last_error_detail(ctypes.byref(d))
        raise HipError(code, msg.decode() if msg else "", d.as_dict() if d.status == code else {})


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p) if a.size else None


class _Buffer:
    def __init__(self, ctx: "HipContext", handle: int):
        self._ctx = ctx
        self._h = _vp(handle)
        ctx._children.add(self)

    @property
    def handle(self):
        return self._h

    def __len__(self) -> int:
        return int(load_library().dmhip_buffer_len(self._h))

    def is_empty(self) -> bool:
        return len(self) == 0

    @property
    def device_ptr(self) -> int:
        return int(load_library().dmhip_buffer_device_ptr(self._h) or 0)

    def write(self, offset: int, data) -> None:
        arr = np.ascontiguousarray(data)
        _check(load_library().dmhip_buffer_write(self._ctx.handle, self._h, offset,
                                                  arr.ctypes.data, arr.nbytes))

    def read(self, offset: int, nbytes: int, dtype=np.uint8) -> np.ndarray:
        out = np.empty(nbytes, dtype=np.uint8)
        _check(load_library().dmhip_buffer_read(self._ctx.handle, self._h, offset,
                                                 out.ctypes.data, nbytes))
        return out.view(dtype)

    def free(self) -> None:
        if self._h:
            load_library().dmhip_buffer_free(self._h)
            self._h = _vp(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class OwnedBuffer(_Buffer):
    """MetalOwnedBuffer (src/metal.rs:213-243): zero-filled device bytes."""

    def as_bytes(self) -> np.ndarray:
        return self.read(0, len(self))


class MappedBuffer(_Buffer):
    """MetalMappedBuffer (src/metal.rs:207-211, :280-288): a GGUF mapping
    uploaded to HBM once, offsets unchanged."""


class SlotBuffer(OwnedBuffer):
    """An expert slot's gate_up or down bytes, owned by the cache: the
    &MetalOwnedBuffer the reference's with_expert closure receives
    (src/expert.rs:138-164).  Valid while the slot is acquired; never freed
    here."""

    def __init__(self, ctx: "HipContext", handle: int):
        self._ctx = ctx
        self._h = _vp(handle)

    def free(self) -> None:
        self._h = _vp(None)


class HipContext:
    """MetalContext (src/metal.rs:179-1560) on one HIP device."""

    def __init__(self, device: int = 0):
        lib = load_library()
        # Buffers and caches made from this context; close() frees them first.
        self._children = weakref.WeakSet()
        h = _vp()
        _check(lib.dmhip_context_new(device, ctypes.byref(h)))
        self._h = h

    @classmethod
    def new(cls, device: int = 0) -> "HipContext":
        return cls(device)

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            for child in list(self._children):
                child.free()
            load_library().dmhip_context_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- device, buffers ------------------------------------------------------
    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _check(load_library().dmhip_device_name(self._h, buf, 256))
        return buf.value.decode()

    def synchronize(self) -> None:
        _check(load_library().dmhip_synchronize(self._h))

    def map_read_only(self, mapping) -> MappedBuffer:
        arr = np.ascontiguousarray(np.frombuffer(mapping, dtype=np.uint8) if isinstance(mapping, (bytes, bytearray)) else mapping).view(np.uint8)
        h = _vp()
        _check(load_library().dmhip_map_read_only(self._h, arr.ctypes.data if arr.size else None,
                                                   arr.size, ctypes.byref(h)))
        return MappedBuffer(self, h.value)

    def new_owned_buffer(self, length: int) -> OwnedBuffer:
        h = _vp()
        _check(load_library().dmhip_new_owned_buffer(self._h, length, ctypes.byref(h)))
        return OwnedBuffer(self, h.value)

    def device_array(self, data) -> OwnedBuffer:
        """An owned buffer holding a copy of `data` (helper for device APIs)."""
        arr = np.ascontiguousarray(data)
        buf = self.new_owned_buffer(max(arr.nbytes, 1))
        if arr.nbytes:
            buf.write(0, arr)
        return buf

    def copy_to_host(self, device_ptr: int, nbytes: int, dtype=np.uint8) -> np.ndarray:
        out = np.empty(nbytes, dtype=np.uint8)
        _check(load_library().dmhip_copy_to_host(self._h, out.ctypes.data, device_ptr, nbytes))
        return out.view(dtype)

    def copy_to_device(self, device_ptr: int, data) -> None:
        arr = np.ascontiguousarray(data)
        _check(load_library().dmhip_copy_to_device(self._h, device_ptr, arr.ctypes.data, arr.nbytes))

    # -- host-slice operators --------------------------------------------------
    def rms_norm(self, input, weight, epsilon: float, output: np.ndarray) -> None:
        x = _f32(input)
        w = None if weight is None else _f32(weight)
        _check(load_library().dmhip_rms_norm(self._h, _fp(x), x.size, None if w is None else _fp(w),
                                             0 if w is None else w.size, epsilon, _fp(output), output.size))

    def silu_mul(self, gate, up, output: np.ndarray) -> None:
        g, u = _f32(gate), _f32(up)
        _check(load_library().dmhip_silu_mul(self._h, _fp(g), g.size, _fp(u), u.size, _fp(output), output.size))

    def softcap(self, input, cap: float, output: np.ndarray) -> None:
        """MetalContext::softcap (src/metal.rs:600-622)."""
        x = _f32(input)
        _check(load_library().dmhip_softcap(self._h, _fp(x), x.size, cap, _fp(output), output.size))

    def add(self, left, right, output: np.ndarray) -> None:
        """MetalContext::add (src/metal.rs:404-432)."""
        a, b = _f32(left), _f32(right)
        _check(load_library().dmhip_add(self._h, _fp(a), a.size, _fp(b), b.size, _fp(output), output.size))

    def gelu_mul(self, gate, up, output: np.ndarray) -> None:
        """MetalContext::gelu_mul (src/metal.rs:530-552)."""
        g, u = _f32(gate), _f32(up)
        _check(load_library().dmhip_gelu_mul(self._h, _fp(g), g.size, _fp(u), u.size, _fp(output), output.size))

    def softmax(self, input, output: np.ndarray) -> None:
        """MetalContext::softmax (src/metal.rs:578-598)."""
        x = _f32(input)
        _check(load_library().dmhip_softmax(self._h, _fp(x), x.size, _fp(output), output.size))

    def rope_neox_in_place(self, values: np.ndarray, heads: int, head_dimension: int, rotated_pairs: int,
                           position: int, theta: float) -> None:
        """MetalContext::rope_neox_in_place (src/metal.rs:478-528): `values`
        (float32, contiguous) is rotated in place."""
        if not (isinstance(values, np.ndarray) and values.dtype == np.float32 and values.flags.c_contiguous):
            raise TypeError("rope_neox_in_place rotates a contiguous float32 array in place")
        _check(load_library().dmhip_rope_neox_in_place(self._h, _fp(values), values.size, heads, head_dimension,
                                                       rotated_pairs, position, theta))

    def argmax(self, input) -> int:
        x = _f32(input)
        idx = ctypes.c_size_t()
        _check(load_library().dmhip_argmax(self._h, _fp(x), x.size, ctypes.byref(idx)))
        return idx.value

    def top_k_softmax(self, logits, k: int) -> list[tuple[int, float]]:
        x = _f32(logits)
        ids = np.zeros(max(k, 1), dtype=np.uintp)
        probs = np.zeros(max(k, 1), dtype=np.float32)
        _check(load_library().dmhip_top_k_softmax(self._h, _fp(x), x.size, k, ids.ctypes.data_as(_szp),
                                                  _fp(probs)))
        return [(int(ids[i]), float(probs[i])) for i in range(k)]

    def matvec(self, kind: int, rows: int, columns: int, encoded, input, output: np.ndarray) -> None:
        enc = np.ascontiguousarray(encoded, dtype=np.uint8)
        x = _f32(input)
        _check(load_library().dmhip_matvec(self._h, kind, rows, columns,
                                           enc.ctypes.data_as(_u8p) if enc.size else None, enc.size,
                                           _fp(x), x.size, _fp(output), output.size))

    def matvec_mapped(self, kind, rows, columns, mapping: MappedBuffer, offset, length, input,
                      output: np.ndarray) -> None:
        x = _f32(input)
        _check(load_library().dmhip_matvec_mapped(self._h, kind, rows, columns, mapping.handle, offset,
                                                  length, _fp(x), x.size, _fp(output), output.size))

    def matvec_owned(self, kind, rows, columns, encoded: OwnedBuffer, offset, length, input,
                     output: np.ndarray) -> None:
        x = _f32(input)
        _check(load_library().dmhip_matvec_owned(self._h, kind, rows, columns, encoded.handle, offset,
                                                 length, _fp(x), x.size, _fp(output), output.size))

    def dequantize(self, kind: int, encoded: _Buffer, offset: int, length: int, elements: int) -> np.ndarray:
        out = np.zeros(max(elements, 1), dtype=np.float32)
        _check(load_library().dmhip_dequantize(self._h, kind, encoded.handle, offset, length,
                                               _fp(out), elements))
        return out[:elements]

    # -- device operators (device addresses as ints) ------------------------
    def matvec_device(self, kind, rows, columns, w_ptr, batch, x_ptr, y_ptr) -> None:
        _check(load_library().dmhip_matvec_device(self._h, kind, rows, columns, w_ptr, batch, x_ptr, y_ptr))

    def matvec_batch_device(self, kind, rows, columns, w_ptrs, x_ptr, x_stride, y_ptr, y_stride) -> None:
        """y + i*y_stride = W_i . (x + i*x_stride) for each device address in w_ptrs."""
        arr = (_vp * max(len(w_ptrs), 1))(*w_ptrs)
        _check(load_library().dmhip_matvec_batch_device(self._h, kind, rows, columns, len(w_ptrs), arr, x_ptr,
                                                        x_stride, y_ptr, y_stride))

    def matvec_argmax_device(self, kind, rows, columns, w_ptr, x_ptr, y_ptr, index_ptr) -> None:
        _check(load_library().dmhip_matvec_argmax_device(self._h, kind, rows, columns, w_ptr, x_ptr,
                                                         y_ptr, index_ptr))

    def argmax_result(self) -> int:
        idx = ctypes.c_size_t()
        _check(load_library().dmhip_argmax_result(self._h, ctypes.byref(idx)))
        return idx.value

    def rms_norm_device(self, batch, count, x_ptr, w_ptr, eps, y_ptr) -> None:
        _check(load_library().dmhip_rms_norm_device(self._h, batch, count, x_ptr, w_ptr, eps, y_ptr))

    def silu_mul_device(self, count, g_ptr, u_ptr, out_ptr) -> None:
        _check(load_library().dmhip_silu_mul_device(self._h, count, g_ptr, u_ptr, out_ptr))

    def softcap_device(self, count, in_ptr, cap, out_ptr) -> None:
        _check(load_library().dmhip_softcap_device(self._h, count, in_ptr, cap, out_ptr))

    def add_device(self, count, a_ptr, b_ptr, out_ptr) -> None:
        _check(load_library().dmhip_add_device(self._h, count, a_ptr, b_ptr, out_ptr))

    def gelu_mul_device(self, count, g_ptr, u_ptr, out_ptr) -> None:
        _check(load_library().dmhip_gelu_mul_device(self._h, count, g_ptr, u_ptr, out_ptr))

    def rope_neox_device(self, v_ptr, values_len, heads, head_dimension, rotated_pairs, position, theta) -> None:
        _check(load_library().dmhip_rope_neox_device(self._h, v_ptr, values_len, heads, head_dimension,
                                                     rotated_pairs, position, theta))

    def ffn_workspace_bytes(self, batch, hidden, ffn) -> int:
        return int(load_library().dmhip_ffn_workspace_bytes(batch, hidden, ffn))

    def ffn_device(self, batch, hidden, ffn, gate_type, gate_ptr, up_type, up_ptr, down_type,
                   down_ptr, eps, h_ptr, y_ptr, ws_ptr, ws_len) -> None:
        _check(load_library().dmhip_ffn_device(self._h, batch, hidden, ffn, gate_type, gate_ptr, up_type,
                                               up_ptr, down_type, down_ptr, eps, h_ptr, y_ptr, ws_ptr, ws_len))

    @staticmethod
    def ffn_noalloc_scratch_bytes() -> int:
        return int(load_library().dmhip_ffn_noalloc_scratch_bytes())

    def ffn_device_noalloc(self, batch, hidden, ffn, gate_type, gate_ptr, up_type, up_ptr, down_type, down_ptr,
                           eps, h_ptr, y_ptr) -> None:
        """ffn_device without a workspace (the library's fixed per-device scratch)."""
        _check(load_library().dmhip_ffn_device_noalloc(self._h, batch, hidden, ffn, gate_type, gate_ptr, up_type,
                                                       up_ptr, down_type, down_ptr, eps, h_ptr, y_ptr))

    def router_top_k_device(self, batch, hidden, experts, k, router_ptr, x_ptr, logits_ptr, ids_ptr,
                            probs_ptr) -> None:
        _check(load_library().dmhip_router_top_k_device(self._h, batch, hidden, experts, k, router_ptr,
                                                        x_ptr, logits_ptr, ids_ptr, probs_ptr))

    def router_result(self) -> None:
        """Raises NonFinite when the last router_top_k_device saw a non-finite logit."""
        _check(load_library().dmhip_router_result(self._h))

    def gemm_workspace_bytes(self, m, k) -> int:
        return int(load_library().dmhip_gemm_workspace_bytes(m, k))

    def gemm_device(self, kind, m, n, k, a_ptr, w_ptr, c_ptr, ws_ptr, ws_len) -> None:
        _check(load_library().dmhip_gemm_device(self._h, kind, m, n, k, a_ptr, w_ptr, c_ptr, ws_ptr, ws_len))

    def event_record(self) -> int:
        ev = _vp()
        _check(load_library().dmhip_event_record(self._h, ctypes.byref(ev)))
        return ev.value

    @staticmethod
    def event_elapsed_ms(start: int, stop: int) -> float:
        ms = ctypes.c_float()
        _check(load_library().dmhip_event_elapsed_ms(_vp(start), _vp(stop), ctypes.byref(ms)))
        return ms.value

    def copy_device(self, dst_ptr: int, src_ptr: int, nbytes: int) -> None:
        _check(load_library().dmhip_copy_device(self._h, dst_ptr, src_ptr, nbytes))

    @staticmethod
    def event_free(ev: int) -> None:
        load_library().dmhip_event_free(_vp(ev))

    # -- GLM safetensors matrices (src/metal.rs:738-1146) ---------------------
    def matvec_safetensor_mapped(self, dtype: str, rows: int, columns: int, mapping: MappedBuffer, offset: int,
                                 length: int, scale, input, output: np.ndarray) -> None:
        """`scale` is None or (MappedBuffer, offset, length)."""
        x = _f32(input)
        sm, so, sl = (None, 0, 0) if scale is None else (scale[0].handle, scale[1], scale[2])
        _check(load_library().dmhip_matvec_safetensor_mapped(self._h, SAFE[dtype], rows, columns, mapping.handle,
                                                             offset, length, sm, so, sl, _fp(x), x.size,
                                                             _fp(output), output.size))

    def matvec_safetensor(self, dtype: str, rows: int, columns: int, encoded, scales, input,
                          output: np.ndarray) -> None:
        enc = np.ascontiguousarray(encoded, dtype=np.uint8)
        sc = None if scales is None else _f32(scales)
        x = _f32(input)
        _check(load_library().dmhip_matvec_safetensor(
            self._h, SAFE[dtype], rows, columns, enc.ctypes.data_as(_u8p) if enc.size else None, enc.size,
            None if sc is None else (_fp(sc) if sc.size else ctypes.cast(ctypes.c_void_p(8), _f32p)),
            0 if sc is None else sc.size, _fp(x), x.size, _fp(output), output.size))

    def matvec_safetensor_device(self, dtype: str, rows, columns, w_ptr, w_len, s_ptr, s_len, x_ptr, y_ptr) -> None:
        _check(load_library().dmhip_matvec_safetensor_device(self._h, SAFE[dtype], rows, columns, w_ptr, w_len,
                                                             s_ptr, s_len, x_ptr, y_ptr))

    # -- attention over a KV ring (src/metal.rs:1196-1511) --------------------
    def new_kv_layer(self, width: int, max_context: int, sliding_window: int | None) -> "KvLayer":
        h = _vp()
        _check(load_library().dmhip_new_kv_layer(self._h, width, max_context, int(sliding_window is not None),
                                                  sliding_window or 0, ctypes.byref(h)))
        return KvLayer(self, h.value)

    def append_kv(self, layer: "KvLayer", position: int, key, value) -> None:
        k, v = _f32(key), _f32(value)
        _check(load_library().dmhip_append_kv(self._h, layer.handle, position, _fp(k), k.size, _fp(v), v.size))

    def append_kv_device(self, layer: "KvLayer", position: int, key_ptr, key_len, value_ptr, value_len) -> None:
        _check(load_library().dmhip_append_kv_device(self._h, layer.handle, position, key_ptr, key_len,
                                                     value_ptr, value_len))

    def attention_cached(self, query, cache: "KvLayer", query_heads: int, kv_heads: int, head_dimension: int,
                         output: np.ndarray) -> None:
        q = _f32(query)
        _check(load_library().dmhip_attention_cached(self._h, _fp(q), q.size, cache.handle, query_heads,
                                                     kv_heads, head_dimension, _fp(output), output.size))

    def attention_cached_device(self, q_ptr, query_len, cache: "KvLayer", query_heads, kv_heads, head_dimension,
                                out_ptr, output_len) -> None:
        _check(load_library().dmhip_attention_cached_device(self._h, q_ptr, query_len, cache.handle, query_heads,
                                                            kv_heads, head_dimension, out_ptr, output_len))

    def attention_result(self) -> None:
        _check(load_library().dmhip_attention_result(self._h))

    def attention(self, query, keys, values, query_heads: int, kv_heads: int, head_dimension: int,
                  window: int | None, output: np.ndarray) -> None:
        q, k, v = _f32(query), _f32(keys), _f32(values)
        _check(load_library().dmhip_attention(self._h, _fp(q), q.size, _fp(k), k.size, _fp(v), v.size,
                                              query_heads, kv_heads, head_dimension, int(window is not None),
                                              window or 0, _fp(output), output.size))

    # -- routed experts -------------------------------------------------------
    def moe_layer(self, cache: "ExpertCache", layer, batch, hidden, width, experts, k, router_ptr,
                  gate_up_type, down_type, x_ptr, y_ptr):
        ids = np.zeros(batch * k, dtype=np.uint32)
        probs = np.zeros(batch * k, dtype=np.float32)
        _check(load_library().dmhip_moe_layer(self._h, cache.handle, layer, batch, hidden, width, experts,
                                              k, router_ptr, gate_up_type, down_type, x_ptr, y_ptr,
                                              ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                              _fp(probs)))
        return ids.reshape(batch, k).astype(np.int64), probs.reshape(batch, k)


class KvLayer:
    """MetalKvLayer (src/metal.rs:245-277): a device KV ring of one layer."""

    def __init__(self, ctx: HipContext, handle: int):
        self._ctx = ctx
        self._h = _vp(handle)
        ctx._children.add(self)

    @property
    def handle(self):
        return self._h

    def position(self) -> int:
        return load_library().dmhip_kv_layer_position(self._h)

    def capacity(self) -> int:
        return load_library().dmhip_kv_layer_capacity(self._h)

    def allocated_bytes(self) -> int:
        return load_library().dmhip_kv_layer_allocated_bytes(self._h)

    def clear(self) -> None:
        load_library().dmhip_kv_layer_clear(self._h)

    def truncate(self, position: int) -> None:
        load_library().dmhip_kv_layer_truncate(self._h, position)

    def width(self) -> int:
        return load_library().dmhip_kv_layer_width(self._h)

    def keys_ptr(self) -> int:
        return load_library().dmhip_kv_layer_keys(self._h)

    def values_ptr(self) -> int:
        return load_library().dmhip_kv_layer_values(self._h)

    def free(self) -> None:
        if getattr(self, "_h", None):
            load_library().dmhip_kv_layer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedHostBuffer:
    """Page-locked host memory (hipHostMalloc) exposed as a numpy array."""

    def __init__(self, nbytes: int):
        p = _vp()
        _check(load_library().dmhip_host_alloc_pinned(nbytes, ctypes.byref(p)))
        self._p = p
        self.nbytes = nbytes
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(p.value))

    @property
    def address(self) -> int:
        return self._p.value

    def free(self):
        if self._p:
            self.array = None
            load_library().dmhip_host_free_pinned(self._p)
            self._p = _vp(None)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass(frozen=True)
class ExpertLayerLayout:
    """src/expert.rs:44-51."""
    expert_count: int
    gate_up_offset: int
    gate_up_bytes: int
    down_offset: int
    down_bytes: int


class ExpertCache:
    """ExpertCache (src/expert.rs:64-229): per-layer LRU of HBM slots filled
    by asynchronous uploads, from host memory (`source` an array or a
    PinnedHostBuffer) or from a file (`file`: an object with fileno(), or a
    descriptor), as the reference's Arc<File>."""

    def __init__(self, ctx: HipContext, source, layouts: Sequence[ExpertLayerLayout], slots_per_layer: int,
                 file=None):
        self._ctx = ctx
        lay = (_Layout * max(len(layouts), 1))()
        for i, l in enumerate(layouts):
            lay[i] = _Layout(l.expert_count, l.gate_up_offset, l.gate_up_bytes, l.down_offset, l.down_bytes)
        h = _vp()
        if file is not None:
            self._source = file  # keeps the descriptor's owner alive
            fd = file if isinstance(file, int) else file.fileno()
            _check(load_library().dmhip_expert_cache_new_file(ctx.handle, fd, lay, len(layouts), slots_per_layer,
                                                              ctypes.byref(h)))
        else:
            if isinstance(source, PinnedHostBuffer):
                self._source = source
                addr, n = source.address, source.nbytes
            else:
                arr = np.ascontiguousarray(source, dtype=np.uint8)
                self._source = arr
                addr, n = arr.ctypes.data, arr.size
            _check(load_library().dmhip_expert_cache_new(ctx.handle, addr, n, lay, len(layouts), slots_per_layer,
                                                         ctypes.byref(h)))
        self._h = h
        ctx._children.add(self)

    @classmethod
    def from_file(cls, ctx: HipContext, file, layouts: Sequence[ExpertLayerLayout], slots_per_layer: int):
        return cls(ctx, None, layouts, slots_per_layer, file=file)

    @property
    def handle(self):
        return self._h

    def slots_per_layer(self) -> int:
        return int(load_library().dmhip_expert_cache_slots_per_layer(self._h))

    def stats(self) -> dict:
        s = _Stats()
        _check(load_library().dmhip_expert_cache_stats_get(self._h, ctypes.byref(s)))
        return {n: getattr(s, n) for n, _ in _Stats._fields_}

    def acquire(self, layer: int, expert: int, cancelled: bool = False):
        """dmhip_expert_acquire: (slot, gate_up SlotBuffer, down SlotBuffer),
        the slot pinned until release()."""
        flag = ctypes.c_int(1 if cancelled else 0)
        slot = ctypes.c_size_t()
        gu = _vp()
        dn = _vp()
        _check(load_library().dmhip_expert_acquire(self._h, layer, expert, ctypes.byref(flag),
                                                   ctypes.byref(slot), ctypes.byref(gu), ctypes.byref(dn)))
        return slot.value, SlotBuffer(self._ctx, gu.value), SlotBuffer(self._ctx, dn.value)

    def release(self, layer: int, slot: int) -> None:
        _check(load_library().dmhip_expert_release(self._h, layer, slot))

    def with_expert(self, layer: int, expert: int, cancelled: Callable[[], bool], use_expert):
        """src/expert.rs:138-164: cancellation checked before and after the
        acquire; the slot stays pinned while `use_expert(gate_up, down)`
        (the slot's SlotBuffers) enqueues its work."""
        if cancelled():
            raise HipError(22, "expert loading was cancelled")
        slot, gu, dn = self.acquire(layer, expert, False)
        try:
            if cancelled():
                raise HipError(22, "expert loading was cancelled")
            return use_expert(gu, dn)
        finally:
            self.release(layer, slot)

    def free(self):
        if getattr(self, "_h", None):
            load_library().dmhip_expert_cache_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class BackendSelection:
    """BackendSelection::from_environment (src/runtime.rs:152-186) with the
    `hip` arm this backend adds: DISKMULE_BACKEND=auto|hip|cpu."""

    CPU = "cpu"
    HIP = "hip"

    @staticmethod
    def from_environment(env=None) -> str:
        env = os.environ if env is None else env
        requested = env.get("DISKMULE_BACKEND", "auto")
        if requested == "cpu":
            return BackendSelection.CPU
        if requested in ("auto", "hip"):
            if os.path.exists(_LIB) and (requested == "hip" or _device_present()):
                return BackendSelection.HIP
            if requested == "hip":
                raise HipError(24, "DISKMULE_BACKEND=hip requires libdmhip.so and a HIP device")
            return BackendSelection.CPU
        raise HipError(24, "DISKMULE_BACKEND must be auto, hip, or cpu")


def _device_present() -> bool:
    return os.path.exists("/dev/kfd")
