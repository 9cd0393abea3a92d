"""The Qwen3.5 matvec offload through the raw C ABI, in the order the
reference's graph makes its calls (src/qwen35/metal.rs:25-50):

  Qwen35MetalWeights::new    -> MetalContext::new     = dmhip_context_new(0)
                             -> map_read_only(mmap)   = dmhip_map_read_only(whole file)
  Qwen35MetalWeights::matvec -> matvec_mapped(kind, dims[1], dims[0], mapping,
                                              absolute_offset, byte_len, x, y)
                             =  dmhip_matvec_mapped(...)

over a GGUF v3 file written and memory-mapped here (tests/gguf_file.py), one
tensor of each type the path serves plus a norm vector.  The host-side checks
of Qwen35MetalWeights::matvec (index past the table -> Overflow, rank != 2 ->
UnsupportedTensorType) run before any library call, as in the reference.
Outputs are checked against the oracle's sequential-fma matvec."""
import ctypes
import mmap

import numpy as np
import pytest

from diskmule_amd import synth
from diskmule_amd.hip import load_library
from oracle import capi
from tests import gguf_file
from tests.tolerance import assert_close

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0, Q5_0, F16, F32 = 12, 14, 8, 6, 1, 0
MATRICES = [("blk.0.attn_q.weight", Q4_K, 512, 1024), ("blk.0.ffn_down.weight", Q6_K, 1024, 768),
            ("blk.0.ffn_gate.weight", Q8_0, 768, 1024), ("blk.0.attn_v.weight", Q5_0, 128, 1024),
            ("blk.0.ssm_out.weight", F16, 1024, 256), ("blk.0.ssm_alpha.weight", F32, 48, 1024),
            ("output.weight", Q6_K, 3000, 1024)]


class Qwen35Weights:
    """Qwen35MetalWeights (src/qwen35/metal.rs:9-50) over the raw C ABI."""

    def __init__(self, lib, path):
        self.lib = lib
        self.file = open(path, "rb")
        self.mapping = mmap.mmap(self.file.fileno(), 0, access=mmap.ACCESS_READ)
        self.bytes = np.frombuffer(self.mapping, np.uint8)
        self.tensors = gguf_file.read_tensors(self.mapping)
        self.ctx = ctypes.c_void_p()
        assert lib.dmhip_context_new(0, ctypes.byref(self.ctx)) == 0, lib.dmhip_last_error()
        self.buf = ctypes.c_void_p()
        code = lib.dmhip_map_read_only(self.ctx, self.bytes.ctypes.data, self.bytes.size, ctypes.byref(self.buf))
        assert code == 0, lib.dmhip_last_error()

    def matvec(self, index, x, y):
        if index >= len(self.tensors):
            return "Overflow"
        t = self.tensors[index]
        if len(t.dimensions) != 2:
            return "UnsupportedTensorType"
        f32p = ctypes.POINTER(ctypes.c_float)
        return self.lib.dmhip_matvec_mapped(self.ctx, t.kind, t.dimensions[1], t.dimensions[0], self.buf,
                                            t.absolute_offset, t.byte_len, x.ctypes.data_as(f32p), x.size,
                                            y.ctypes.data_as(f32p), y.size)

    def close(self):
        self.lib.dmhip_buffer_free(self.buf)
        self.lib.dmhip_context_free(self.ctx)
        del self.bytes
        self.mapping.close()
        self.file.close()


def test_qwen35_matvec_sequence_over_a_mapped_gguf(tmp_path):
    tensors, encoded = [], {}
    for i, (name, kind, rows, cols) in enumerate(MATRICES):
        w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(400 + i, kind))
        encoded[name] = w
        tensors.append((name, [cols, rows], kind, w.tobytes()))
    norm = synth.normal(synth.activation_seed(499), 1024).astype(np.float32)
    tensors.insert(3, ("blk.0.attn_norm.weight", [1024], F32, norm.tobytes()))
    path = tmp_path / "qwen35-small.gguf"
    gguf_file.write(path, tensors)

    lib = load_library()
    weights = Qwen35Weights(lib, path)
    try:
        names = [t.name for t in weights.tensors]
        for i, t in enumerate(weights.tensors):
            print("tensor", t.name, t.kind, t.dimensions, t.absolute_offset, flush=True)
            cols = t.dimensions[0]
            rows = t.dimensions[1] if len(t.dimensions) == 2 else 1
            x = synth.normal(synth.activation_seed(450 + i), cols).astype(np.float32)
            y = np.zeros(rows, np.float32)
            status = weights.matvec(i, x, y)
            if len(t.dimensions) != 2:
                assert status == "UnsupportedTensorType"
                continue
            assert status == 0, lib.dmhip_last_error()
            want = capi.matvec(t.kind, rows, cols, encoded[t.name], x)
            assert_close(y, want, t.name)
        assert weights.matvec(len(names), np.zeros(1, np.float32), np.zeros(1, np.float32)) == "Overflow"
        # a wrong-length activation is the library's InvalidInputLength (13)
        t = weights.tensors[0]
        y = np.zeros(t.dimensions[1], np.float32)
        assert weights.matvec(0, np.zeros(t.dimensions[0] - 1, np.float32), y) == 13
    finally:
        weights.close()
