"""Pins the oracle's GLM safetensors matrices (orc_st_*, src/glm52/cpu.rs:
1180-1420 and u8_matrix_encoding, src/metal.rs:1893-1942) before the GPU is
checked against it: the reference's own known answers, the E4M3FN format's
published landmark values over all 256 patterns, and an exact-rational brute
force of the product-then-sum fold."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import capi


def f32(v):
    return np.float32(v)


# ---- the reference's known answers -------------------------------------------

def test_row_int8_and_grouped_int4_known_answers():
    # src/glm52/cpu.rs:1551-1606
    i8 = np.array([-127, 0, 127, -2, 3, 4], dtype=np.int8).view(np.uint8)
    assert capi.st_u8_encoding(2, 3, 6, 8)["format"] == capi.ST_INT8_ROW
    out = capi.st_matvec(capi.ST_INT8_ROW, 2, 3, i8, [0.1, 0.5], [1.0, 2.0, -1.0])
    assert out.tolist() == [f32(-25.4), 0.0]
    assert capi.st_dequantize_row(capi.ST_INT8_ROW, 2, 3, i8, [0.1, 0.5], 1).tolist() == [-1.0, 1.5, 2.0]
    i4 = [0x40, 0xC8, 0x0F, 0xA9, 0xCB, 0x0D]
    enc = capi.st_u8_encoding(2, 5, 6, 8)
    assert enc == {"format": capi.ST_INT4_GROUPED, "group_size": 5, "scale_columns": 1}
    out = capi.st_matvec(capi.ST_INT4_GROUPED, 2, 5, i4, [0.5, 2.0], [1.0] * 5, group_size=5)
    assert out.tolist() == [-0.5, 30.0]
    row = capi.st_dequantize_row(capi.ST_INT4_GROUPED, 2, 5, i4, [0.5, 2.0], 0, group_size=5)
    assert row.tolist() == [-4.0, -2.0, 0.0, 2.0, 3.5]


def test_metal_fixture_values():
    # src/metal.rs:2315-2404: BF16 2x3 and F8_E4M3FN 129x130 with 2x2 block scales
    bf16 = np.array([1.0, 2.0, 3.0, -1.0, 0.5, 4.0], dtype=np.float32).view(np.uint32) >> 16
    enc = bf16.astype("<u2").view(np.uint8)
    out = capi.st_matvec(capi.ST_BF16, 2, 3, enc, None, [2.0, -1.0, 0.5])
    assert np.abs(out - [1.5, -0.5]).max() <= 1e-6
    fp8 = np.full(129 * 130, 0x38, dtype=np.uint8)
    x = np.ones(130, dtype=np.float32)
    x[129] = 2.0
    out = capi.st_matvec(capi.ST_F8_E4M3, 129, 130, fp8, [2.0, 3.0, 5.0, 7.0], x)
    assert np.abs(out[:128] - 265.0).max() <= 1e-5 and abs(out[128] - 661.0) < 1e-5
    # src/metal.rs:2406-2486: grouped INT4, 33 columns, group 16 (three scales per row)
    int4 = np.full(2 * 17, 0x99, dtype=np.uint8)
    enc = capi.st_u8_encoding(2, 33, 34, 24)
    assert enc == {"format": capi.ST_INT4_GROUPED, "group_size": 16, "scale_columns": 3}
    out = capi.st_matvec(capi.ST_INT4_GROUPED, 2, 33, int4, [1.0, 2.0, 4.0, 0.5, 1.0, 2.0], np.ones(33),
                         group_size=16)
    assert np.abs(out - [52.0, 26.0]).max() <= 1e-5


def test_flat_layout_that_is_neither_encoding_is_rejected():
    # src/glm52/cpu.rs:1603-1606: 196 bytes against 256 columns
    r = capi.st_u8_encoding(1, 256, 196, 4)
    assert r["error"] == capi.INVALID_BYTE_LENGTH and (r["expected"], r["actual"]) == (128, 196)


# ---- E4M3FN over all 256 patterns -----------------------------------------------

LANDMARKS = {0x38: 1.0, 0xC0: -2.0, 0x7E: 448.0, 0xFE: -448.0, 0x08: 2.0 ** -6, 0x07: 7 * 2.0 ** -9,
             0x01: 2.0 ** -9, 0x00: 0.0, 0x3C: 1.5, 0x77: 240.0, 0x78: 256.0}


def test_f8_e4m3fn_landmarks_and_every_pattern():
    for bits, want in LANDMARKS.items():
        assert capi.st_decode_f8(bits) == want, hex(bits)
    assert capi.st_decode_f8(0x7F) is None and capi.st_decode_f8(0xFF) is None
    neg_zero = capi.st_decode_f8(0x80)
    assert neg_zero == 0.0 and np.signbit(neg_zero)
    values = []
    for bits in range(256):
        v = capi.st_decode_f8(bits)
        if bits & 0x7F == 0x7F:
            continue
        values.append(v)
        # sign symmetry, and magnitudes strictly increasing with the code
        assert capi.st_decode_f8(bits ^ 0x80) == -v
    pos = [capi.st_decode_f8(b) for b in range(0x7F)]
    assert all(a < b for a, b in zip(pos, pos[1:]))
    # spacing: 8 values per binade above the subnormals, step 2^-9 below 2^-6
    assert all(pos[i + 1] - pos[i] == 2.0 ** -9 for i in range(8))
    for e in range(1, 15):
        lo = 2.0 ** (e - 7)
        assert pos[8 * e] == lo and pos[8 * e + 7] == lo * 1.875


# ---- exact-rational fold ---------------------------------------------------------

def rounded(v: Fraction) -> Fraction:
    return Fraction(float(np.float32(float(v))))


@pytest.mark.parametrize("fmt", [capi.ST_BF16, capi.ST_F8_E4M3, capi.ST_INT8_ROW, capi.ST_INT4_GROUPED])
def test_product_then_sum_fold_brute_force(fmt):
    rng = np.random.default_rng(fmt + 10)
    rows, cols, group = 3, 70, 32
    if fmt == capi.ST_BF16:
        enc = (rng.standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype("<u2").view(np.uint8)
        scales = None
    elif fmt == capi.ST_F8_E4M3:
        enc = rng.integers(0, 256, rows * cols).astype(np.uint8)
        enc[(enc & 0x7F) == 0x7F] = 0x38
        scales = rng.uniform(0.5, 2.0, 1).astype(np.float32)
    elif fmt == capi.ST_INT8_ROW:
        enc = rng.integers(0, 256, rows * cols).astype(np.uint8)
        scales = rng.uniform(0.01, 0.1, rows).astype(np.float32)
    else:
        enc = rng.integers(0, 256, rows * ((cols + 1) // 2)).astype(np.uint8)
        scales = rng.uniform(0.01, 0.1, rows * ((cols + group - 1) // group)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    out = capi.st_matvec(fmt, rows, cols, enc, scales, x, group_size=group)
    for r in range(rows):
        w = capi.st_dequantize_row(fmt, rows, cols, enc, scales, r, group_size=group)
        acc = Fraction(0)
        for c in range(cols):
            acc = rounded(acc + rounded(Fraction(float(w[c])) * Fraction(float(x[c]))))
        assert float(acc) == float(out[r])


def test_dequantized_weights_follow_the_formats():
    # each weight is one f32 product of the decoded code and its scale
    rng = np.random.default_rng(4)
    rows, cols = 130, 260
    enc = rng.integers(0, 0x7F, rows * cols).astype(np.uint8) | (rng.integers(0, 2, rows * cols) << 7).astype(np.uint8)
    sc = rng.uniform(0.5, 2.0, 2 * 3).astype(np.float32)
    table = np.array([capi.st_decode_f8(b) if b & 0x7F != 0x7F else np.nan for b in range(256)], np.float32)
    for r in (0, 127, 128, 129):
        row = capi.st_dequantize_row(capi.ST_F8_E4M3, rows, cols, enc, sc, r)
        want = table[enc[r * cols:(r + 1) * cols]] * sc[(r // 128) * 3 + np.arange(cols) // 128]
        assert np.array_equal(row, want.astype(np.float32))
    i4 = rng.integers(0, 256, rows * 130).astype(np.uint8)
    sc4 = rng.uniform(0.5, 2.0, rows * 3).astype(np.float32)
    row = capi.st_dequantize_row(capi.ST_INT4_GROUPED, rows, cols, i4, sc4, 5, group_size=96)
    nib = np.stack([i4[5 * 130:6 * 130] & 15, i4[5 * 130:6 * 130] >> 4], 1).ravel()
    assert np.array_equal(row, ((nib.astype(np.float32) - 8) * sc4[5 * 3 + np.arange(cols) // 96]).astype(np.float32))


@pytest.mark.parametrize("cols,scale_len,group", [(256, 4 * 16, 16), (256, 4 * 8, 32), (240, 4 * 5, 48),
                                                  (256, 4 * 4, 64), (288, 4 * 3, 96), (256, 4 * 2, 128),
                                                  (384, 4 * 2, 192), (512, 4 * 2, 256), (100, 4, 100)])
def test_u8_encoding_group_sizes(cols, scale_len, group):
    r = capi.st_u8_encoding(1, cols, (cols + 1) // 2, scale_len)
    assert r == {"format": capi.ST_INT4_GROUPED, "group_size": group, "scale_columns": -(-cols // group)}


def test_u8_encoding_errors():
    r = capi.st_u8_encoding(2, 64, 64, 12)  # int4 bytes, 3 scales: no group size fits
    assert r["error"] == capi.INVALID_BYTE_LENGTH and r["scales"] and (r["expected"], r["actual"]) == (8, 12)
    assert capi.st_u8_encoding(2 ** 62, 8, 0, 0)["error"] == capi.OVERFLOW
    # a group size larger than the row stops the search (16 > 8 columns)
    r = capi.st_u8_encoding(1, 8, 4, 8)
    assert r["error"] == capi.INVALID_BYTE_LENGTH and r["scales"]
