"""Affine group-64 quantization (8- and 4-bit codes), dequantization and GEMM (numpy, CPU).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates the quantized-linear arithmetic the reference gets from nn.quantize /
nn.QuantizedLinear (src/mlx_dspark/load.py:204-206, :285-286; target layers reached from
src/mlx_dspark/target.py:66-74): w = scale * q + bias per group of 64 input columns, with
bf16 scale and bias. MLX's own quantizer rounding is external and unpinned; the engine
documents its own rule (include/dspark_hip.h, dsk_w8_quantize) and this module restates it.

Pinning: quantize -> dequantize round trip is within scale/2 per element (closed form);
dequantized GEMM vs a float64 brute-force dot product on tiny shapes; the GPU quantizer is
compared bit for bit against quantize() below.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest even), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize(w: np.ndarray, bits: int = 8):
    """w [N, K] float32 -> (q uint8 [N, K], scale bf16-bits [N, K/64], bias bf16-bits [N, K/64]);
    codes 0 .. 2^bits - 1 (bits 8 or 4), s = (max - min) / (2^bits - 1)."""
    levels = np.float32((1 << bits) - 1)
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    g = w.reshape(N, K // 64, 64)
    lo = g.min(axis=2)
    hi = g.max(axis=2)
    s = (hi - lo) / levels
    s16 = bf16_bits(s)
    sf = bits_to_f32(s16)
    bad = ~(sf > 0)
    s16 = np.where(bad, np.uint16(0x3F80), s16)
    sf = np.where(bad, np.float32(1.0), sf)
    b16 = bf16_bits(lo)
    bf = bits_to_f32(b16)
    t = np.rint((g - bf[..., None]) / sf[..., None])
    q = np.clip(t, 0, levels).astype(np.uint8).reshape(N, K)
    return q, s16, b16


def dequantize(q: np.ndarray, s16: np.ndarray, b16: np.ndarray) -> np.ndarray:
    N, K = q.shape
    s = bits_to_f32(s16).astype(np.float64)
    b = bits_to_f32(b16).astype(np.float64)
    w = q.reshape(N, K // 64, 64).astype(np.float64) * s[..., None] + b[..., None]
    return w.reshape(N, K)


def gemm(x: np.ndarray, q, s16, b16) -> np.ndarray:
    """y = x . deq(W)^T in float64 (x already in the activation dtype's values)."""
    return np.asarray(x, dtype=np.float64) @ dequantize(q, s16, b16).T
