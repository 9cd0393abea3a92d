"""Vectorised numpy restatement of the GGUF block decoders.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

This is the *second*, independent restatement used to cross-check the C
oracle.  The C oracle follows ``src/cpu.rs:546-645``; this module follows the
indexing of the reference's Metal kernels instead (``metal/kernels.metal``:
``q4_k_scale``/``q4_k_minimum`` :20-32, ``matvec_q8_0`` :377-396,
``matvec_q4_k`` :398-434, ``matvec_q6_k`` :436-484), with every float32
operation done by numpy in float32 (correctly rounded, never fused), and the
f16 widening done by numpy's own float16 -> float32 conversion.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 6, 8, 12, 14, 30


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _le16(block: np.ndarray, offset: int) -> np.ndarray:
    return block[:, offset].astype(np.uint16) | (block[:, offset + 1].astype(np.uint16) << 8)


def q4_k_scale(scales: np.ndarray, index: int) -> np.ndarray:
    """kernels.metal:20-25 (scales: [blocks, 12] uint8)."""
    if index < 4:
        return scales[:, index] & 0x3F
    return (scales[:, index + 4] & 0x0F) | ((scales[:, index - 4] >> 6) << 4)


def q4_k_minimum(scales: np.ndarray, index: int) -> np.ndarray:
    """kernels.metal:27-32."""
    if index < 4:
        return scales[:, index + 4] & 0x3F
    return (scales[:, index + 4] >> 4) | ((scales[:, index] >> 6) << 4)


def decode_q4_k(encoded: np.ndarray) -> np.ndarray:
    blocks = np.asarray(encoded, dtype=np.uint8).reshape(-1, 144)
    delta = f16_bits_to_f32(_le16(blocks, 0))
    minimum = f16_bits_to_f32(_le16(blocks, 2))
    scales = blocks[:, 4:16]
    quants = blocks[:, 16:144]
    out = np.empty((blocks.shape[0], 256), dtype=np.float32)
    for group_pair in range(4):
        scale_low = delta * q4_k_scale(scales, 2 * group_pair).astype(np.float32)
        min_low = minimum * q4_k_minimum(scales, 2 * group_pair).astype(np.float32)
        scale_high = delta * q4_k_scale(scales, 2 * group_pair + 1).astype(np.float32)
        min_high = minimum * q4_k_minimum(scales, 2 * group_pair + 1).astype(np.float32)
        packed = quants[:, 32 * group_pair: 32 * group_pair + 32]
        base = 64 * group_pair
        out[:, base: base + 32] = scale_low[:, None] * (packed & 0x0F).astype(np.float32) - min_low[:, None]
        out[:, base + 32: base + 64] = scale_high[:, None] * (packed >> 4).astype(np.float32) - min_high[:, None]
    return out.reshape(-1)


def decode_q6_k(encoded: np.ndarray) -> np.ndarray:
    blocks = np.asarray(encoded, dtype=np.uint8).reshape(-1, 210)
    delta = f16_bits_to_f32(_le16(blocks, 208))
    out = np.empty((blocks.shape[0], 256), dtype=np.float32)
    index = np.arange(32)
    scale_pair = index // 16
    for half in range(2):
        low = blocks[:, half * 64: half * 64 + 64]
        high = blocks[:, 128 + half * 32: 128 + half * 32 + 32]
        sc = blocks[:, 192 + half * 8: 192 + half * 8 + 8].view(np.int8).astype(np.float32)
        base = half * 128
        q1 = (low[:, index] & 0x0F) | ((high[:, index] & 0x03) << 4)
        q2 = (low[:, index + 32] & 0x0F) | (((high[:, index] >> 2) & 0x03) << 4)
        q3 = (low[:, index] >> 4) | (((high[:, index] >> 4) & 0x03) << 4)
        q4 = (low[:, index + 32] >> 4) | (((high[:, index] >> 6) & 0x03) << 4)
        for q, off, sp in ((q1, 0, 0), (q2, 32, 2), (q3, 64, 4), (q4, 96, 6)):
            scale = delta[:, None] * sc[:, scale_pair + sp]
            out[:, base + off: base + off + 32] = scale * (q.astype(np.float32) - np.float32(32.0))
    return out.reshape(-1)


def decode_q8_0(encoded: np.ndarray) -> np.ndarray:
    blocks = np.asarray(encoded, dtype=np.uint8).reshape(-1, 34)
    delta = f16_bits_to_f32(_le16(blocks, 0))
    quants = blocks[:, 2:34].view(np.int8).astype(np.float32)
    return (delta[:, None] * quants).reshape(-1)


def decode_q5_0(encoded: np.ndarray) -> np.ndarray:
    """kernels.metal:346-375 indexing."""
    blocks = np.asarray(encoded, dtype=np.uint8).reshape(-1, 22)
    delta = f16_bits_to_f32(_le16(blocks, 0))
    high_bits = (blocks[:, 2].astype(np.uint32) | (blocks[:, 3].astype(np.uint32) << 8)
                 | (blocks[:, 4].astype(np.uint32) << 16) | (blocks[:, 5].astype(np.uint32) << 24))
    out = np.empty((blocks.shape[0], 32), dtype=np.float32)
    for index in range(16):
        packed = blocks[:, 6 + index].astype(np.uint32)
        low_high = ((high_bits >> index) << 4) & 0x10
        high_high = (high_bits >> (index + 12)) & 0x10
        low = ((packed & 0x0F) | low_high).astype(np.int32) - 16
        high = ((packed >> 4) | high_high).astype(np.int32) - 16
        out[:, index] = delta * low.astype(np.float32)
        out[:, index + 16] = delta * high.astype(np.float32)
    return out.reshape(-1)


def dequantize(ggml_type: int, encoded) -> np.ndarray:
    enc = np.asarray(encoded, dtype=np.uint8)
    if ggml_type == Q4_K:
        return decode_q4_k(enc)
    if ggml_type == Q6_K:
        return decode_q6_k(enc)
    if ggml_type == Q8_0:
        return decode_q8_0(enc)
    if ggml_type == Q5_0:
        return decode_q5_0(enc)
    if ggml_type == F16:
        return f16_bits_to_f32(enc.view(np.uint16))
    if ggml_type == F32:
        return enc.view(np.float32).copy()
    if ggml_type == BF16:
        return (enc.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise ValueError(f"unsupported type {ggml_type}")
