"""Seeded synthetic inputs for the quantized-matrix path.

The generator is SplitMix64 as the reference's sampler defines it
(``src/runtime.rs:1017-1031``): ``state += 0x9e3779b97f4a7c15`` then the
two xor-shift-multiply rounds.  Because the state only advances by a
constant, the i-th output is ``mix(seed + (i + 1) * gamma)``, so numpy can
draw any counter range without iterating.

Block contents follow the BASELINE configurations:

* Q4_K (144 B): ``d ~ U(1e-4, 2e-3)`` and ``dmin ~ U(0, 1e-3)`` as f16,
  then 12 scale bytes and 128 quant bytes uniform.  Block ``j`` uses draws
  ``[20 j, 20 j + 20)``: draw 0 -> d, draw 1 -> dmin, draws 2..19 -> bytes.
* Q6_K (210 B): 128 + 64 uniform quant bytes, 16 int8 scales ``U{-32..31}``,
  ``d ~ U(1e-4, 1e-3)`` as f16.  Block ``j`` uses draws ``[28 j, 28 j + 28)``:
  draw 0 -> d, draws 1..24 -> quant bytes, draws 25..26 -> scales.
* Q8_0 (34 B): ``d ~ U(1e-3, 1e-2)`` as f16 and 32 uniform int8.  Block
  ``j`` uses draws ``[6 j, 6 j + 6)``.
* f32 activations ~ N(0, 1) by Box-Muller on pairs of draws.
* bf16 values by round-to-nearest-even from f32.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

# ggml type ids (src/gguf.rs:295-318)
F32, F16, Q5_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 6, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34),
         Q4_K: (256, 144), Q6_K: (256, 210)}


def weight_seed(config: int, tensor: int = 0) -> int:
    return (0xD15C0000 + config) | (tensor << 32)


def activation_seed(config: int, tensor: int = 0) -> int:
    return (0xD15C1000 + config) | (tensor << 32)


def row_bytes(ggml_type: int, columns: int) -> int:
    elems, nbytes = BLOCK[ggml_type]
    if columns % elems:
        raise ValueError(f"{columns} columns is not a multiple of the {elems}-element block")
    return columns // elems * nbytes


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs ``start .. start+count`` of SplitMix64 seeded with ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def unit(draws: np.ndarray) -> np.ndarray:
    """``(next >> 11) * 2^-53`` as in ``src/runtime.rs:1028-1030``."""
    return (draws >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def _f16_bits(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint16)


def q4_k_blocks(seed: int, blocks: int, chunk: int = 1 << 19) -> np.ndarray:
    out = np.empty((blocks, 144), dtype=np.uint8)
    for b0 in range(0, blocks, chunk):
        nb = min(chunk, blocks - b0)
        d = splitmix64(seed, 20 * b0, 20 * nb).reshape(nb, 20)
        out[b0:b0 + nb, 0:2] = _f16_bits(1e-4 + (2e-3 - 1e-4) * unit(d[:, 0]))[:, None].view(np.uint8)
        out[b0:b0 + nb, 2:4] = _f16_bits(1e-3 * unit(d[:, 1]))[:, None].view(np.uint8)
        raw = np.ascontiguousarray(d[:, 2:20]).view(np.uint8)  # 144 bytes, little endian
        out[b0:b0 + nb, 4:144] = raw[:, :140]
    return out.reshape(-1)


def q6_k_blocks(seed: int, blocks: int, chunk: int = 1 << 19) -> np.ndarray:
    out = np.empty((blocks, 210), dtype=np.uint8)
    for b0 in range(0, blocks, chunk):
        nb = min(chunk, blocks - b0)
        d = splitmix64(seed, 28 * b0, 28 * nb).reshape(nb, 28)
        out[b0:b0 + nb, 0:192] = np.ascontiguousarray(d[:, 1:25]).view(np.uint8)
        sc = np.ascontiguousarray(d[:, 25:27]).view(np.uint8)
        out[b0:b0 + nb, 192:208] = ((sc & 63).astype(np.int16) - 32).astype(np.int8).view(np.uint8)
        out[b0:b0 + nb, 208:210] = _f16_bits(1e-4 + (1e-3 - 1e-4) * unit(d[:, 0]))[:, None].view(np.uint8)
    return out.reshape(-1)


def q8_0_blocks(seed: int, blocks: int, chunk: int = 1 << 20) -> np.ndarray:
    out = np.empty((blocks, 34), dtype=np.uint8)
    for b0 in range(0, blocks, chunk):
        nb = min(chunk, blocks - b0)
        d = splitmix64(seed, 6 * b0, 6 * nb).reshape(nb, 6)
        out[b0:b0 + nb, 0:2] = _f16_bits(1e-3 + 9e-3 * unit(d[:, 0]))[:, None].view(np.uint8)
        out[b0:b0 + nb, 2:34] = np.ascontiguousarray(d[:, 1:5]).view(np.uint8)
    return out.reshape(-1)


def q5_0_blocks(seed: int, blocks: int, chunk: int = 1 << 20) -> np.ndarray:
    """Q5_0 blocks (d, 32 high bits, 16 nibble bytes) with random codes."""
    out = np.empty((blocks, 22), dtype=np.uint8)
    for b0 in range(0, blocks, chunk):
        nb = min(chunk, blocks - b0)
        d = splitmix64(seed, 4 * b0, 4 * nb).reshape(nb, 4)
        out[b0:b0 + nb, 0:2] = _f16_bits(1e-3 + 9e-3 * unit(d[:, 0]))[:, None].view(np.uint8)
        out[b0:b0 + nb, 2:22] = np.ascontiguousarray(d[:, 1:4]).view(np.uint8)[:, :20]
    return out.reshape(-1)


def quantized_matrix(ggml_type: int, rows: int, columns: int, seed: int) -> np.ndarray:
    """Row-major encoded matrix: ``rows`` rows of ``columns`` values."""
    elems, _ = BLOCK[ggml_type]
    blocks = rows * (columns // elems)
    if ggml_type == Q4_K:
        return q4_k_blocks(seed, blocks)
    if ggml_type == Q6_K:
        return q6_k_blocks(seed, blocks)
    if ggml_type == Q8_0:
        return q8_0_blocks(seed, blocks)
    if ggml_type == Q5_0:
        return q5_0_blocks(seed, blocks)
    if ggml_type == F32:
        return normal(seed, rows * columns).view(np.uint8)
    if ggml_type == F16:
        return _f16_bits(normal(seed, rows * columns)).view(np.uint8)
    raise ValueError(f"no generator for type {ggml_type}")


def normal(seed: int, count: int, start: int = 0) -> np.ndarray:
    d = splitmix64(seed, 2 * start, 2 * count)
    u1 = 1.0 - unit(d[0::2])
    u2 = unit(d[1::2])
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (finite inputs)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + np.uint64(0x7FFF) + ((bits >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
