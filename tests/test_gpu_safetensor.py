"""GPU parity of the GLM safetensors matvecs (MetalContext::matvec_safetensor
and _mapped, src/metal.rs:738-1146) through the C ABI: the reference's own
known answers, every E4M3FN code through both kernels, the oracle
(src/glm52/cpu.rs:1180-1420 semantics) on seeded matrices within a rounding
bound, the reference's validation errors in its order, and the device entry
point against the host one."""
import numpy as np
import pytest

from diskmule_amd import HipError
from oracle import capi
from tests.tolerance import assert_close

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
ST = {"BF16": capi.ST_BF16, "F8_E4M3": capi.ST_F8_E4M3}


def expect_error(variant, fn, *args, **detail):
    with pytest.raises(HipError) as e:
        fn(*args)
    assert e.value.variant == variant, str(e.value)
    for k, v in detail.items():
        assert e.value.detail.get(k) == v, (k, e.value.detail)
    return e.value


def bf16_bytes(values):
    bits = np.asarray(values, dtype=np.float32).view(np.uint32) >> 16
    return bits.astype("<u2").view(np.uint8)


# ---- the reference's known answers -----------------------------------------------

def test_row_int8_and_grouped_int4_known_answers(ctx):
    # src/glm52/cpu.rs:1551-1606 through the host-slice entry point
    i8 = np.array([-127, 0, 127, -2, 3, 4], dtype=np.int8).view(np.uint8)
    out = np.zeros(2, dtype=np.float32)
    ctx.matvec_safetensor("U8", 2, 3, i8, [0.1, 0.5], [1.0, 2.0, -1.0], out)
    assert out.tolist() == [np.float32(-25.4), 0.0]
    i4 = np.array([0x40, 0xC8, 0x0F, 0xA9, 0xCB, 0x0D], dtype=np.uint8)
    ctx.matvec_safetensor("U8", 2, 5, i4, [0.5, 2.0], [1.0] * 5, out)
    assert out.tolist() == [-0.5, 30.0]


def test_mapped_bf16_and_fp8_match_cpu_values(ctx):
    # src/metal.rs:2315-2404, the same file layout and offsets
    bf16 = bf16_bytes([1.0, 2.0, 3.0, -1.0, 0.5, 4.0])
    fp8 = np.full(129 * 130, 0x38, dtype=np.uint8)
    bf16_offset, fp8_offset = 32, 64
    scale_offset = fp8_offset + fp8.size + 2
    scales = np.array([2.0, 3.0, 5.0, 7.0], dtype=np.float32)
    contents = np.zeros(scale_offset + 16, dtype=np.uint8)
    contents[bf16_offset:bf16_offset + bf16.size] = bf16
    contents[fp8_offset:fp8_offset + fp8.size] = fp8
    contents[scale_offset:scale_offset + 16] = scales.view(np.uint8)
    mapped = ctx.map_read_only(contents)
    out = np.zeros(2, dtype=np.float32)
    ctx.matvec_safetensor_mapped("BF16", 2, 3, mapped, bf16_offset, bf16.size, None, [2.0, -1.0, 0.5], out)
    assert np.abs(out - [1.5, -0.5]).max() <= 1e-6
    ctx.matvec_safetensor("BF16", 2, 3, bf16, None, [2.0, -1.0, 0.5], out)
    assert np.abs(out - [1.5, -0.5]).max() <= 1e-6
    x = np.ones(130, dtype=np.float32)
    x[129] = 2.0
    out = np.zeros(129, dtype=np.float32)
    ctx.matvec_safetensor_mapped("F8_E4M3", 129, 130, mapped, fp8_offset, fp8.size, (mapped, scale_offset, 16), x,
                                 out)
    assert np.abs(out[:128] - 265.0).max() <= 1e-5 and abs(out[128] - 661.0) < 1e-5
    ctx.matvec_safetensor("F8_E4M3", 129, 130, fp8, scales, x, out)
    assert np.abs(out[:128] - 265.0).max() <= 1e-5 and abs(out[128] - 661.0) < 1e-5


def test_mapped_and_owned_u8_matvecs_match_reference_values(ctx):
    # src/metal.rs:2406-2486: row INT8 and grouped INT4 (33 columns, group 16)
    int8 = np.array([-127, 0, 127, -2, 3, 4], dtype=np.int8).view(np.uint8)
    int8_scales = np.array([0.1, 0.5], dtype=np.float32)
    int4 = np.full(2 * 17, 0x99, dtype=np.uint8)
    int4_scales = np.array([1.0, 2.0, 4.0, 0.5, 1.0, 2.0], dtype=np.float32)
    int8_offset = 33
    int8_scale_offset = int8_offset + int8.size + 5
    int4_offset = int8_scale_offset + 8 + 7
    int4_scale_offset = int4_offset + int4.size + 3
    contents = np.zeros(int4_scale_offset + 24, dtype=np.uint8)
    contents[int8_offset:int8_offset + 6] = int8
    contents[int8_scale_offset:int8_scale_offset + 8] = int8_scales.view(np.uint8)
    contents[int4_offset:int4_offset + int4.size] = int4
    contents[int4_scale_offset:int4_scale_offset + 24] = int4_scales.view(np.uint8)
    mapped = ctx.map_read_only(contents)
    out = np.zeros(2, dtype=np.float32)
    ctx.matvec_safetensor_mapped("U8", 2, 3, mapped, int8_offset, 6, (mapped, int8_scale_offset, 8),
                                 [1.0, 2.0, -1.0], out)
    assert np.abs(out - [-25.4, 0.0]).max() <= 1e-5
    ctx.matvec_safetensor_mapped("U8", 2, 33, mapped, int4_offset, int4.size, (mapped, int4_scale_offset, 24),
                                 np.ones(33), out)
    assert np.abs(out - [52.0, 26.0]).max() <= 1e-5
    ctx.matvec_safetensor("U8", 2, 33, int4, int4_scales, np.ones(33), out)
    assert np.abs(out - [52.0, 26.0]).max() <= 1e-5


# ---- every E4M3FN code through both kernels ----------------------------------------

@pytest.mark.parametrize("columns", [16, 17])  # 16: the wide kernel (hardware converter); 17: the generic one
def test_every_f8_code_decodes_as_the_reference(ctx, columns):
    rows = 256
    enc = np.zeros((rows, columns), dtype=np.uint8)
    enc[:, 0] = np.arange(256)
    x = np.zeros(columns, dtype=np.float32)
    x[0] = 1.0
    scales = np.ones(2 * 1, dtype=np.float32)
    out = np.zeros(rows, dtype=np.float32)
    ctx.matvec_safetensor("F8_E4M3", rows, columns, enc.ravel(), scales, x, out)
    for code in range(256):
        want = capi.st_decode_f8(code)
        if want is None:
            assert np.isnan(out[code]), hex(code)  # metal/kernels.metal:264-266
        else:
            assert out[code] == want, (hex(code), out[code], want)


# ---- seeded parity against the oracle ------------------------------------------------

def make(fmt, rows, cols, group, rng):
    if fmt == "BF16":
        return bf16_bytes(rng.standard_normal(rows * cols) * 0.05), None, capi.ST_BF16
    if fmt == "F8_E4M3":
        enc = rng.integers(0, 256, rows * cols).astype(np.uint8)
        enc[(enc & 0x7F) == 0x7F] = 0x38
        sc = rng.uniform(1e-3, 4e-3, (-(-rows // 128)) * (-(-cols // 128))).astype(np.float32)
        return enc, sc, capi.ST_F8_E4M3
    if fmt == "I8":
        enc = rng.integers(0, 256, rows * cols).astype(np.uint8)
        return enc, rng.uniform(1e-3, 1e-2, rows).astype(np.float32), capi.ST_INT8_ROW
    enc = rng.integers(0, 256, rows * ((cols + 1) // 2)).astype(np.uint8)
    sc = rng.uniform(1e-3, 1e-2, rows * (-(-cols // group))).astype(np.float32)
    return enc, sc, capi.ST_INT4_GROUPED


def bound(fmt_id, rows, cols, enc, sc, group, x):
    """Per-row rounding budget: both evaluations sum cols products in fp32
    (the GPU in chunks with its scale factored out of each chunk, the INT4
    chunks as sum(n x) - 8 sum(x))."""
    b = np.zeros(rows)
    ax = np.abs(x.astype(np.float64))
    for r in range(rows):
        w = capi.st_dequantize_row(fmt_id, rows, cols, enc, sc, r, group_size=group).astype(np.float64)
        s = np.abs(w) @ ax
        if fmt_id == capi.ST_INT4_GROUPED:
            cs = sc[r * (-(-cols // group)) + np.arange(cols) // group].astype(np.float64)
            s += 8.0 * (cs @ ax)
        b[r] = 4.0 * (cols + 64) * U * s + 1e-30
    return b


CASES = [
    ("BF16", 4096, 4096, 0), ("BF16", 300, 1000, 0), ("BF16", 257, 129, 0),
    ("F8_E4M3", 6144, 2048, 0), ("F8_E4M3", 300, 1040, 0), ("F8_E4M3", 129, 130, 0),
    ("I8", 4096, 4096, 0), ("I8", 200, 1008, 0), ("I8", 70, 99, 0),
    ("I4", 2048, 6144, 32), ("I4", 512, 4096, 16), ("I4", 512, 4096, 128), ("I4", 300, 2048, 4096 // 2),
    ("I4", 130, 960, 48), ("I4", 64, 257, 64), ("I4", 200, 1024, 1024),
]


@pytest.mark.parametrize("fmt,rows,cols,group", CASES)
def test_seeded_parity(ctx, fmt, rows, cols, group):
    print(f"safetensor {fmt} {rows}x{cols} group {group}", flush=True)
    rng = np.random.default_rng(rows * 31 + cols + group)
    if fmt == "I4" and group == 4096 // 2:
        group = cols  # one scale per row
    enc, sc, fmt_id = make(fmt, rows, cols, group, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    out = np.zeros(rows, dtype=np.float32)
    ctx.matvec_safetensor("U8" if fmt in ("I8", "I4") else fmt, rows, cols, enc, sc, x, out)
    want = capi.st_matvec(fmt_id, rows, cols, enc, sc, x, group_size=group)
    assert_close(out, want, f"{fmt} {rows}x{cols}")
    diff = np.abs(out.astype(np.float64) - want)
    b = bound(fmt_id, rows, cols, enc, sc, group, x)
    assert (diff <= b).all(), f"{fmt}: worst {float((diff / b).max()):.3f}x the bound"


def test_device_entry_point_matches_the_host_one(ctx):
    rng = np.random.default_rng(5)
    for fmt, rows, cols, group in (("F8_E4M3", 1024, 2048, 0), ("I4", 1024, 2048, 32), ("I8", 513, 2048, 0),
                                   ("BF16", 512, 2048, 0)):
        enc, sc, _ = make(fmt, rows, cols, group, rng)
        x = rng.standard_normal(cols).astype(np.float32)
        dtype = "U8" if fmt in ("I8", "I4") else fmt
        host = np.zeros(rows, dtype=np.float32)
        ctx.matvec_safetensor(dtype, rows, cols, enc, sc, x, host)
        wb, xb, yb = ctx.device_array(enc), ctx.device_array(x), ctx.new_owned_buffer(rows * 4)
        sb = ctx.device_array(sc) if sc is not None else None
        ctx.matvec_safetensor_device(dtype, rows, cols, wb.device_ptr, enc.size, sb.device_ptr if sb else None,
                                     0 if sc is None else sc.size, xb.device_ptr, yb.device_ptr)
        got = yb.read(0, rows * 4, np.float32)
        assert np.array_equal(got.view(np.uint32), host.view(np.uint32)), fmt
        for b in (wb, xb, yb, sb):
            if b is not None:
                b.free()


def test_f32_and_f16_go_through_the_gguf_path(ctx):
    rng = np.random.default_rng(9)
    w = rng.standard_normal((64, 256)).astype(np.float32)
    x = rng.standard_normal(256).astype(np.float32)
    out = np.zeros(64, dtype=np.float32)
    ctx.matvec_safetensor("F32", 64, 256, w.view(np.uint8).ravel(), None, x, out)
    assert_close(out, w.astype(np.float64) @ x, "F32")
    h = w.astype(np.float16)
    ctx.matvec_safetensor("F16", 64, 256, h.view(np.uint8).ravel(), None, x, out)
    assert_close(out, h.astype(np.float64) @ x, "F16")


def test_zero_rows_is_a_no_op(ctx):
    out = np.zeros(0, dtype=np.float32)
    ctx.matvec_safetensor("BF16", 0, 8, np.zeros(0, np.uint8), None, np.ones(8), out)
    ctx.matvec_safetensor("U8", 0, 8, np.zeros(0, np.uint8), np.zeros(0, np.float32), np.ones(8), out)


# ---- validation, in src/metal.rs's order -----------------------------------------------

def test_host_checks(ctx):
    out2 = np.zeros(2, dtype=np.float32)
    e = expect_error("UnsupportedTensorType", ctx.matvec_safetensor, "I32", 2, 4, np.zeros(32, np.uint8), None,
                     np.ones(4), out2)
    assert e.detail == {"kind": "safetensors dtype"}
    expect_error("InvalidInputLength", ctx.matvec_safetensor, "BF16", 2, 4, np.zeros(16, np.uint8), None,
                 np.ones(3), out2, expected=4, actual=3)
    expect_error("InvalidOutputLength", ctx.matvec_safetensor, "BF16", 2, 4, np.zeros(16, np.uint8), None,
                 np.ones(4), np.zeros(3, np.float32), expected=2, actual=3)
    expect_error("InvalidByteLength", ctx.matvec_safetensor, "BF16", 2, 4, np.zeros(15, np.uint8), None,
                 np.ones(4), out2, kind="BF16", expected=16, actual=15)
    expect_error("InvalidByteLength", ctx.matvec_safetensor, "F8_E4M3", 2, 4, np.zeros(9, np.uint8), None,
                 np.ones(4), out2, kind="F8_E4M3FN", expected=8, actual=9)
    expect_error("InvalidVectorLength", ctx.matvec_safetensor, "F8_E4M3", 2, 4, np.zeros(8, np.uint8), None,
                 np.ones(4), out2, operation="F8_E4M3FN matvec", argument="scales", expected=1, actual=0)
    expect_error("InvalidVectorLength", ctx.matvec_safetensor, "F8_E4M3", 2, 4, np.zeros(8, np.uint8),
                 np.ones(2), np.ones(4), out2, operation="F8_E4M3FN matvec", expected=1, actual=2)
    expect_error("EmptyInput", ctx.matvec_safetensor, "BF16", 2, 0, np.zeros(0, np.uint8), None, np.ones(0), out2,
                 operation="safetensors matvec")
    expect_error("InvalidVectorLength", ctx.matvec_safetensor, "U8", 2, 4, np.zeros(8, np.uint8), None,
                 np.ones(4), out2, operation="safetensors U8 matvec", argument="scales", expected=2, actual=0)
    expect_error("InvalidByteLength", ctx.matvec_safetensor, "U8", 2, 4, np.zeros(5, np.uint8), np.ones(2),
                 np.ones(4), out2, kind="U8 quantized matrix", expected=4, actual=5)
    expect_error("InvalidByteLength", ctx.matvec_safetensor, "U8", 2, 64, np.zeros(64, np.uint8), np.ones(3),
                 np.ones(64), out2, kind="U8 quantization scales", expected=8, actual=12)
    expect_error("EmptyInput", ctx.matvec_safetensor, "U8", 2, 0, np.zeros(0, np.uint8), np.ones(2), np.ones(0),
                 out2, operation="safetensors U8 matvec")


def test_mapped_checks(ctx):
    contents = np.zeros(64, dtype=np.uint8)
    mapped = ctx.map_read_only(contents)
    out2 = np.zeros(2, dtype=np.float32)
    expect_error("MappedRange", ctx.matvec_safetensor_mapped, "BF16", 2, 4, mapped, 50, 16, None, np.ones(4), out2,
                 offset=50, end=66, length=64)
    e = expect_error("InvalidByteLength", ctx.matvec_safetensor_mapped, "F8_E4M3", 2, 4, mapped, 0, 8, None,
                     np.ones(4), out2)
    assert e.detail == {"kind": "F8_E4M3FN scale", "expected": 4, "actual": 0}
    expect_error("InvalidByteLength", ctx.matvec_safetensor_mapped, "F8_E4M3", 2, 4, mapped, 0, 8, (mapped, 8, 8),
                 np.ones(4), out2, kind="F8_E4M3FN scale", expected=4, actual=8)
    expect_error("MappedRange", ctx.matvec_safetensor_mapped, "F8_E4M3", 2, 4, mapped, 0, 8, (mapped, 62, 4),
                 np.ones(4), out2, offset=62, end=66, length=64)
    e = expect_error("InvalidByteLength", ctx.matvec_safetensor_mapped, "U8", 2, 4, mapped, 0, 8, None, np.ones(4),
                     out2)
    assert e.detail == {"kind": "U8 quantization scales", "expected": 8, "actual": 0}
    expect_error("MappedRange", ctx.matvec_safetensor_mapped, "U8", 2, 4, mapped, 60, 8, (mapped, 0, 8), np.ones(4),
                 out2, offset=60, end=68, length=64)
