"""CPU checks for the W8 oracle: round-trip bound, brute-force GEMM, degenerate groups."""

import numpy as np
import pytest

from oracle import w8


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_roundtrip_within_half_step(bits):
    rng = np.random.default_rng(bits)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    q, s, b = w8.quantize(w, bits)
    levels = (1 << bits) - 1
    assert q.max() <= levels
    deq = w8.dequantize(q, s, b)
    step = w8.bits_to_f32(s).astype(np.float64)
    err = np.abs(deq - w).reshape(32, 4, 64).max(axis=2)
    # half a step, plus the bf16 rounding of scale and bias (relative 2^-8 of the range)
    assert np.all(err <= step * 0.5 + step * levels * 2**-8 + np.abs(w8.bits_to_f32(b)) * 2**-8 + 1e-9)
    # each group's minimum maps to code 0 and its maximum to the top code (up to bf16 rounding)
    g = q.reshape(32, 4, 64)
    assert np.all(g.min(axis=2) == 0) and np.all(g.max(axis=2) >= levels - 1)


def test_four_bit_codes_on_an_exact_grid():
    """Weights on a 16-level grid with a bf16-exact step come back exactly at 4 bits."""
    codes = np.arange(64) % 16
    w = (0.25 + 0.125 * codes).astype(np.float32)[None, :]
    q, s, b = w8.quantize(w, 4)
    assert np.array_equal(q[0], codes) and w8.bits_to_f32(s)[0, 0] == 0.125 and w8.bits_to_f32(b)[0, 0] == 0.25
    assert np.array_equal(w8.dequantize(q, s, b), w)


def test_constant_group_uses_unit_scale():
    w = np.full((1, 64), 0.5, np.float32)
    q, s, b = w8.quantize(w)
    assert s[0, 0] == 0x3F80 and np.all(q == 0)
    assert np.allclose(w8.dequantize(q, s, b), 0.5)


def test_gemm_matches_bruteforce_dot():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((8, 128)).astype(np.float32)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    q, s, b = w8.quantize(w)
    y = w8.gemm(x, q, s, b)
    sf = w8.bits_to_f32(s).astype(np.float64)
    bf = w8.bits_to_f32(b).astype(np.float64)
    for m in range(3):
        for n in range(8):
            ref = sum(float(x[m, k]) * (sf[n, k // 64] * int(q[n, k]) + bf[n, k // 64]) for k in range(128))
            assert abs(y[m, n] - ref) < 1e-9 * max(1.0, abs(ref))


@pytest.mark.parametrize("bits", [8, 4])
def test_torch_dequant_equals_float64_dequant(bits):
    """The oracle models dequantize with float32 torch ops; that equals the float64 restatement
    rounded to float32, bit for bit (s * q is exact in float32)."""
    import torch

    from oracle.model import deq_codes
    rng = np.random.default_rng(bits)
    N, K = 96, 512
    q = rng.integers(0, 1 << bits, (N, K)).astype(np.uint8)
    scale = (rng.standard_normal((N, K // 64)) * 10.0 ** rng.integers(-6, 1, (N, K // 64))).astype(np.float32)
    bias = (rng.standard_normal((N, K // 64)) * 10.0 ** rng.integers(-6, 1, (N, K // 64))).astype(np.float32)
    s16, b16 = w8.bf16_bits(np.abs(scale)), w8.bf16_bits(bias)
    want = w8.dequantize(q, s16, b16).astype(np.float32)
    st = torch.from_numpy(s16.view(np.int16)).view(torch.bfloat16)
    bt = torch.from_numpy(b16.view(np.int16)).view(torch.bfloat16)
    got = deq_codes(torch.from_numpy(q), st, bt).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
