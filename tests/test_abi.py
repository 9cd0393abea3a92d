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


def test_diagnostics_library_exports_exactly_its_header():
    """The launch-floor probes live in their own library
    (include/dmhip_diag.h), not in the product's exports."""
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "dmhip_diag.h")).read(), flags=re.S)
    declared = set(re.findall(r"\b(dmhip_[a-z0-9_]+)\s*\(", text))
    path = os.path.join(ROOT, "diskmule_amd", "libdmhip_diag.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    assert set(re.findall(r" T (dmhip_\w+)", out)) == declared == {"dmhip_diag_time_empty", "dmhip_diag_time_read"}
    assert not declared & set(header_functions())


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


# ---- the Rust binding (rust/hip.rs) is a transcription of the header --------

def _rust_source():
    return open(os.path.join(ROOT, "rust", "hip.rs")).read()


def _c_struct_fields(name):
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "dmhip.h")).read(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\}" % name, text, flags=re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split()[-1] if "," not in decl else decl
        for part in re.split(r"\s*,\s*", names):
            fields.append(re.sub(r"^.*[\s*]", "", part.strip()))
    return fields


def _rust_struct_fields(name):
    body = re.search(r"pub struct %s \{(.*?)\}" % name, _rust_source(), flags=re.S).group(1)
    return re.findall(r"pub (\w+):", body)


def test_rust_ffi_declares_every_header_function():
    block = _rust_source().split("unsafe extern \"C\" {", 1)[1].split("\n    }\n", 1)[0]
    declared = sorted(set(re.findall(r"pub fn (dmhip_\w+)\(", block)))
    assert declared == sorted(set(header_functions()))


def test_rust_status_constants_match_the_header():
    text = open(os.path.join(ROOT, "include", "dmhip.h")).read()
    c = dict((n, int(v)) for n, v in re.findall(r"(DMHIP_(?:OK|ERR_\w+)) = (\d+)", text))
    rust = dict((n, int(v)) for n, v in re.findall(r"pub const (DMHIP_(?:OK|ERR_\w+)): c_int = (\d+);",
                                                   _rust_source()))
    assert rust == c and len(c) == 32


def test_rust_structs_have_the_header_field_order():
    for name in ("dmhip_error_detail", "dmhip_expert_layer_layout", "dmhip_expert_cache_stats"):
        assert _rust_struct_fields(name) == _c_struct_fields(name), name


def test_rust_type_ids_match_the_header():
    text = open(os.path.join(ROOT, "include", "dmhip.h")).read()
    c = dict((n, int(v)) for n, v in re.findall(r"(DMHIP_TYPE_\w+) = (\d+)", text))
    rust = dict((n, int(v)) for n, v in re.findall(r"pub const (DMHIP_TYPE_\w+): u32 = (\d+);", _rust_source()))
    assert rust == c


def test_gguf_writer_places_tensors_where_the_reference_parser_would():
    from tests import gguf_file
    import tempfile
    data = [("a", [256, 3], 12, bytes(range(144)) * 3), ("b", [7], 0, bytes(28)),
            ("c", [32, 2, 2], 8, bytes(34 * 4))]
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "t.gguf")
        gguf_file.write(path, data, alignment=64)
        blob = open(path, "rb").read()
    infos = gguf_file.read_tensors(blob)
    assert [t.name for t in infos] == ["a", "b", "c"]
    for t, (_, dims, kind, raw) in zip(infos, data):
        assert t.absolute_offset % 64 == 0 and t.dimensions == dims and t.kind == kind
        assert blob[t.absolute_offset:t.absolute_offset + t.byte_len] == raw


def test_every_status_has_a_variant_in_both_bindings():
    text = open(os.path.join(ROOT, "include", "dmhip.h")).read()
    statuses = dict((n, int(v)) for n, v in re.findall(r"(DMHIP_(?:OK|ERR_\w+)) = (\d+)", text))
    from diskmule_amd import hip
    assert sorted(hip.VARIANTS) == sorted(statuses.values())
    src = _rust_source()
    # Command and InvalidArgument fall through to MetalError::Command by design
    for name in set(statuses) - {"DMHIP_OK", "DMHIP_ERR_COMMAND", "DMHIP_ERR_INVALID_ARGUMENT"}:
        assert re.search(r"ffi::%s\b[^=]*=>" % name, src), name


def test_rust_safe_dtype_ids_match_the_header_and_the_python_binding():
    text = open(os.path.join(ROOT, "include", "dmhip.h")).read()
    c = dict((n, int(v)) for n, v in re.findall(r"(DMHIP_SAFE_\w+) = (\d+)", text))
    rust = dict((n, int(v)) for n, v in re.findall(r"pub const (DMHIP_SAFE_\w+): u32 = (\d+);", _rust_source()))
    assert rust == c and len(c) == 15
    from diskmule_amd import hip
    assert {f"DMHIP_SAFE_{k}": v for k, v in hip.SAFE.items()} == c
