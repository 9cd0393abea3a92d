"""CPU checks of the boundary: the C-ABI library loads, exports exactly what
include/dmhip.h declares, and the host-side logic that needs no GPU."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from diskmule_amd import hip, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "dmhip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dmhip_[a-z0-9_]+)\s*\(", text)))


def test_binding_list_matches_header():
    assert sorted(hip.EXPORTED_SYMBOLS) == header_functions()


def test_library_loads_and_exports_every_declared_symbol():
    lib = hip.load_library()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", hip.library_path()], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (dmhip_\w+)", out))
    assert exported == set(header_functions())


def test_library_is_built_for_gfx950_only():
    # The offload bundle of our own build names its target triples.
    blob = open(hip.library_path(), "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-f]+)", blob))
    assert targets == {b"gfx950"}


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_context_without_a_device_reports_no_device():
    with pytest.raises(hip.HipError) as err:
        hip.HipContext(0)
    assert err.value.variant == "NoDevice"


def test_null_arguments_are_rejected_before_any_device_work():
    lib = hip.load_library()
    assert lib.dmhip_context_new(0, None) == 24
    assert lib.dmhip_synchronize(None) == 24
    assert lib.dmhip_buffer_len(None) == 0
    assert b"must not be null" in lib.dmhip_last_error()


def test_backend_selection_mirrors_runtime_rs():
    assert hip.BackendSelection.from_environment({"DISKMULE_BACKEND": "cpu"}) == "cpu"
    with pytest.raises(hip.HipError):
        hip.BackendSelection.from_environment({"DISKMULE_BACKEND": "metal-ish"})
    assert hip.BackendSelection.from_environment({"DISKMULE_BACKEND": "hip"}) == "hip"


# ---- synthetic generator (counter-based SplitMix64) ----------------------

def test_splitmix64_matches_the_sequential_definition():
    # src/runtime.rs:1017-1031, stepped one value at a time
    def seq(seed, n):
        s = seed
        out = []
        for _ in range(n):
            s = (s + 0x9E3779B97F4A7C15) & (2 ** 64 - 1)
            z = s
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2 ** 64 - 1)
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2 ** 64 - 1)
            out.append(z ^ (z >> 31))
        return out
    assert synth.splitmix64(1234, 0, 20).tolist() == seq(1234, 20)
    assert synth.splitmix64(1234, 5, 3).tolist() == seq(1234, 8)[5:]


def test_block_generators_follow_the_configured_distributions():
    w = synth.quantized_matrix(12, 64, 4096, synth.weight_seed(1)).reshape(-1, 144)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dmin = w[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    assert d.min() >= 9.99e-5 and d.max() <= 2.001e-3
    assert dmin.min() >= 0 and dmin.max() <= 1.001e-3
    w6 = synth.quantized_matrix(14, 64, 4096, synth.weight_seed(2)).reshape(-1, 210)
    sc = w6[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d6 = w6[:, 208:210].copy().view(np.float16).astype(np.float32)
    assert d6.min() >= 9.99e-5 and d6.max() <= 1.001e-3
    x = synth.normal(synth.activation_seed(1), 1 << 16)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1) < 0.02
    # chunked generation is the same stream
    a = synth.q4_k_blocks(7, 1000, chunk=64)
    b = synth.q4_k_blocks(7, 1000)
    assert np.array_equal(a, b)


def test_bf16_rounding_is_nearest_even():
    v = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e-3], dtype=np.float32)
    got = synth.bf16_bits_to_f32(synth.to_bf16_bits(v))
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa is 1.0
    assert got.tolist()[:2] == [1.0, 1.0]
    assert got[2] == np.float32(1.015625)
    assert got[3] == -2.5
