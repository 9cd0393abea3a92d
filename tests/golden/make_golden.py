"""Writes the golden fixtures under tests/golden/.

1. ``kat_reference.json``: the known-answer cases of the reference's own unit
   tests, as data (inputs and expected outputs), transcribed from
   ``src/cpu.rs:670-833`` and ``src/expert.rs:266-325`` and
   ``src/metal.rs:2052-2142, :2268-2270`` (the formula-driven matvec
   fixture).  The reference is Rust and cannot be run here; every expected
   value below is the one its test asserts.
2. ``seeded_small.npz``: small seeded inputs (diskmule_amd.synth) with the
   oracle's outputs, used as regression vectors by the GPU parity tests.
   Regenerate after an intentional oracle change only.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def u16le(v: int) -> list[int]:
    return [v & 0xFF, (v >> 8) & 0xFF]


def kat_cases() -> dict:
    cases = {}
    # decodes_f32_and_f16_values (src/cpu.rs:670-687)
    f32_bytes = list(struct.pack("<2f", 1.25, -2.5))
    cases["f32_decode"] = {"type": 0, "encoded": f32_bytes, "expected": [1.25, -2.5]}
    f16_bytes = u16le(0x3C00) + u16le(0xC000) + u16le(0x0001)
    cases["f16_decode"] = {"type": 1, "encoded": f16_bytes, "expected": [1.0, -2.0, 2.0 ** -24]}
    # decodes_q5_0_high_bits_and_nibbles (:689-699)
    block = u16le(0x4000) + [0xFF] * 4 + [0x10] * 16
    cases["q5_0_decode"] = {"type": 6, "encoded": block, "expected": [0.0] * 16 + [2.0] * 16}
    # decodes_q8_0_signed_values (:701-713)
    block = u16le(0x3800) + [((i - 16) & 0xFF) for i in range(32)]
    cases["q8_0_decode"] = {"type": 8, "encoded": block, "expected": [(i - 16.0) * 0.5 for i in range(32)]}
    # decodes_q4_k_group_scales_and_minima (:715-730)
    block = u16le(0x3800) + u16le(0x3400) + [1] * 4 + [2] * 4 + [0x21] * 4 + [0x30] * 128
    cases["q4_k_decode"] = {"type": 12, "encoded": block,
                            "expected": ([-0.5] * 32 + [1.0] * 32) * 4}
    # unpacks_q4_k_high_scale_and_minimum_bits (:732-739)
    scales = [0] * 12
    scales[0], scales[4], scales[8] = 0b1100_0000, 0b1000_0000, 0b1010_0001
    cases["q4_k_scale_min"] = {"index": 4, "scales": scales, "expected": [49, 42]}
    # decodes_q6_k_six_bit_groups (:741-753)
    block = [0] * 192 + [i + 1 for i in range(16)] + u16le(0x3800)
    expected = []
    for g in range(16):
        expected += [-16.0 * (g + 1)] * 16
    cases["q6_k_decode"] = {"type": 14, "encoded": block, "expected": expected}
    # matvec_uses_row_major_tensor_layout (:755-764)
    cases["matvec_row_major"] = {"type": 0, "rows": 2, "columns": 2,
                                 "encoded": list(struct.pack("<4f", 1.0, 2.0, 3.0, 4.0)),
                                 "input": [0.5, -1.0], "expected": [-1.5, -2.5]}
    # rejects_bad_lengths_and_unsupported_types (:766-776)
    cases["reject_q4_k_element_count"] = {"type": 12, "encoded_len": 144, "elements": 32,
                                          "expected_error": "InvalidElementCount"}
    cases["reject_q5_k_unsupported"] = {"type": 13, "encoded_len": 0, "elements": 0,
                                        "expected_error": "UnsupportedType"}
    # normalizes_weighted_and_unweighted_vectors (:778-795): expected values
    # are the closed forms the test states, evaluated in f32.
    inv = np.float32(1.0) / np.sqrt(np.float32(12.5) + np.float32(1e-6))
    cases["rms_norm"] = {"input": [3.0, 4.0], "epsilon": 1e-6,
                         "expected_unweighted": [float(np.float32(3.0) * inv), float(np.float32(4.0) * inv)],
                         "weight": [2.0, 0.5],
                         "expected_weighted": [float(np.float32(6.0) * inv), float(np.float32(2.0) * inv)],
                         "bad_weight": [1.0], "expected_error": "InvalidVectorLength"}
    # softmax_and_top_k_are_stable_and_deterministic (:819-833)
    cases["softmax_stable"] = {"input": [1000.0, 999.0, "-inf"], "sum": 1.0, "sum_tolerance": 1e-6,
                               "expected_last": 0.0}
    cases["top_k"] = {"logits": [2.0, 3.0, 3.0, 0.0], "k": 2, "expected": [[1, 0.5], [2, 0.5]]}
    cases["argmax_ties"] = {"input": [1.0, 4.0, 4.0], "expected": 1}
    cases["top_k_zero"] = {"logits": [1.0], "k": 0, "expected_error": "InvalidTopK"}
    # bounded_cache_tracks_hits_misses_evictions_and_cancellation
    # (src/expert.rs:266-325)
    cases["expert_lru"] = {
        "source": [1, 2, 3, 4, 5, 6, 7, 8, 11, 12, 13, 14, 15, 16, 17, 18],
        "layout": {"expert_count": 2, "gate_up_offset": 0, "gate_up_bytes": 4,
                   "down_offset": 8, "down_bytes": 4},
        "slots_per_layer": 1,
        "accesses": [[0, 0, [1, 2, 3, 4], [11, 12, 13, 14]],
                     [0, 0, [1, 2, 3, 4], [11, 12, 13, 14]],
                     [0, 1, [5, 6, 7, 8], [15, 16, 17, 18]]],
        "expected_stats": {"hits": 1, "misses": 2, "evictions": 1, "reads": 4, "bytes_read": 16,
                           "resident_bytes": 8},
        "cancelled_access": [0, 0], "expected_error": "Cancelled",
    }
    # matvec_fixture + input formula (src/metal.rs:2052-2142, :2268-2270);
    # the expected outputs are the oracle's (the reference asserts CPU vs
    # Metal within max(5e-4, 2e-5*|cpu|), :2041-2050).
    cases["metal_matvec_fixture"] = {"rows": 3, "types": [0, 1, 6, 8, 12, 14],
                                     "tolerance_abs": 5e-4, "tolerance_rel": 2e-5}
    return cases


def metal_matvec_fixture(kind: int, rows: int):
    """src/metal.rs:2052-2142."""
    if kind == 0:
        columns = 64
        vals = [((i * 17) % 41) * 0.03125 - 0.625 for i in range(rows * columns)]
        return columns, np.frombuffer(struct.pack(f"<{len(vals)}f", *vals), dtype=np.uint8).copy()
    if kind == 1:
        columns = 64
        pats = [0x3000, 0xB400, 0x3800, 0xBC00, 0x3C00, 0x4000]
        return columns, np.array([pats[i % 6] for i in range(rows * columns)], dtype="<u2").view(np.uint8).copy()
    enc = []
    blocks = 3
    for row in range(rows):
        for b in range(blocks):
            if kind == 6:
                blk = u16le(0x3400) + [(i * 29 + row * 47 + b * 13 + 3) & 0xFF for i in range(20)]
            elif kind == 8:
                blk = u16le(0x3000) + [((i * 7 - 101 + row * 11 + b * 17) & 0xFF) for i in range(32)]
            elif kind == 12:
                blk = u16le(0x3000) + u16le(0x2800) + [(i * 19 + row * 31 + b * 43 + 5) & 0xFF for i in range(140)]
            elif kind == 14:
                blk = [(i * 23 + row * 37 + b * 41 + 11) & 0xFF for i in range(192)]
                blk += [((i * 5 - 37 + row * 3 + b * 7) & 0xFF) for i in range(16)]
                blk += u16le(0x2800)
            else:
                raise ValueError(kind)
            enc += blk
    columns = (32 if kind in (6, 8) else 256) * blocks
    return columns, np.array(enc, dtype=np.uint8)


def metal_fixture_input(columns: int) -> np.ndarray:
    """src/metal.rs:2268-2270."""
    return np.array([((i * 11 % 53) - 26.0) * 0.0078125 for i in range(columns)], dtype=np.float32)


def seeded_small() -> dict:
    from diskmule_amd import synth
    from oracle import capi
    out = {}
    for name, kind, rows, cols, cfg in (("q4_k", 12, 48, 1024, 1), ("q6_k", 14, 48, 1024, 2),
                                        ("q8_0", 8, 48, 512, 3), ("q6_k_768", 14, 40, 768, 4)):
        w = synth.quantized_matrix(kind, rows, cols, synth.weight_seed(cfg))
        x = synth.normal(synth.activation_seed(cfg), cols)
        out[f"{name}_encoded"] = w
        out[f"{name}_input"] = x
        # a checksum of the exact dequantized values (bit patterns summed as
        # uint64) instead of the values themselves keeps the fixture small
        deq = capi.dequantize(kind, w, rows * cols)
        out[f"{name}_dequant_checksum"] = np.array([int(deq.view(np.uint32).astype(np.uint64).sum())],
                                                   dtype=np.uint64)
        out[f"{name}_matvec"] = capi.matvec(kind, rows, cols, w, x, threads=1)
        out[f"{name}_shape"] = np.array([kind, rows, cols], dtype=np.int64)
    logits = synth.normal(synth.activation_seed(9), 128)
    out["top_k_logits"] = logits
    sel = capi.top_k_softmax(logits, 8)
    out["top_k_ids"] = np.array([s[0] for s in sel], dtype=np.int64)
    out["top_k_probs"] = np.array([s[1] for s in sel], dtype=np.float32)
    return out


def main() -> None:
    with open(os.path.join(HERE, "kat_reference.json"), "w") as f:
        json.dump(kat_cases(), f, indent=1)
        f.write("\n")
    np.savez_compressed(os.path.join(HERE, "seeded_small.npz"), **seeded_small())
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
