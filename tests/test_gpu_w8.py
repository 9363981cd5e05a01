"""GPU parity: W8 quantizer (bit-exact vs oracle), activation pack and skinny GEMM (vs the
float64 oracle), embedding gather."""

import numpy as np
import pytest
import torch

from oracle import w8 as O

pytestmark = pytest.mark.gpu


def _bf16_vals(x: torch.Tensor) -> np.ndarray:
    return x.float().cpu().numpy()


def test_quantize_bitexact(dev):
    from mlx_dspark.ops import W8Weight
    g = torch.Generator().manual_seed(0)
    w = torch.randn(96, 512, generator=g) * 0.02
    w[3, 64:128] = 0.25                                   # constant group
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    qo, so, bo = O.quantize(w.numpy())
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.view(torch.int16).cpu().numpy().view(np.uint16), so)
    assert np.array_equal(b.view(torch.int16).cpu().numpy().view(np.uint16), bo)


def _mlx_np(q, s, b):
    return (q.cpu().numpy(), s.view(torch.int16).cpu().numpy().view(np.uint16),
            b.view(torch.int16).cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (9, 256, 1024), (16, 6144, 4096), (17, 512, 4096),
                                   (36, 4096, 1024), (64, 128, 3072), (16, 192, 4096), (16, 4096, 12288),
                                   (9, 151936 // 8, 1024)])
def test_gemm_matches_oracle(dev, M, N, K):
    from mlx_dspark.ops import W8Weight, act_pack, w8_gemm
    print(f"gemm M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    x = (torch.randn(M, K, generator=g) * 3.0).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    W = W8Weight.from_mlx(q, s, b)
    a = act_pack(x.to(dev))
    y = w8_gemm(a, W, M, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.gemm(_bf16_vals(x), *_mlx_np(q, s, b))
    err = np.abs(y.cpu().numpy() - ref).max() / np.sqrt((ref ** 2).mean())
    assert err < 2e-4, err


def test_gemm_residual_bf16_softcap_and_norm_modes(dev):
    from mlx_dspark.ops import (DSK_PACK_RMSNORM, DSK_PACK_SILU, W8Weight, act_pack, w8_gemm)
    g = torch.Generator().manual_seed(5)
    M, N, K = 16, 1024, 2048
    w = torch.randn(N, K, generator=g) * 0.02
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    W = W8Weight.from_mlx(q, s, b)
    deq = O.dequantize(*_mlx_np(q, s, b))
    # RMSNorm prologue + bf16 residual in place + softcap
    x = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    res = (torch.randn(M, N, generator=g)).to(torch.bfloat16)
    yd = res.to(dev).clone()
    a = act_pack(x.to(dev), DSK_PACK_RMSNORM, nw.to(dev), 1e-6)
    w8_gemm(a, W, M, out=yd, residual=yd, softcap=30.0)
    xf = x.float().numpy().astype(np.float64)
    xn = xf / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + 1e-6) * nw.float().numpy()
    xn = O.bf16_round(xn.astype(np.float32)).astype(np.float64)
    ref = np.tanh((res.float().numpy() + xn @ deq.T) / 30.0) * 30.0
    got = yd.float().cpu().numpy()
    assert np.abs(got - ref).max() < 0.02 + 0.01 * np.abs(ref).max()
    # SiLU(gate) * up prologue
    gu = (torch.randn(M, 2 * K, generator=g)).to(torch.bfloat16)
    a = act_pack(gu.to(dev), DSK_PACK_SILU, K=K)
    y = w8_gemm(a, W, M, out_dtype=torch.float32)
    gf, uf = gu.float().numpy()[:, :K].astype(np.float64), gu.float().numpy()[:, K:].astype(np.float64)
    act = O.bf16_round((O.bf16_round((gf / (1 + np.exp(-gf))).astype(np.float32)) * uf).astype(np.float32))
    ref2 = act.astype(np.float64) @ deq.T
    err = np.abs(y.cpu().numpy() - ref2).max() / np.sqrt((ref2 ** 2).mean())
    assert err < 5e-3, err


def test_embed_gather(dev):
    from mlx_dspark.ops import W8Table, W8Weight, w8_embed
    g = torch.Generator().manual_seed(2)
    V, H = 1000, 256
    w = torch.randn(V, H, generator=g) * 0.02
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    t = W8Table(q, s, b)
    ids = torch.tensor([0, 5, 999, 5, 123], dtype=torch.int32, device=dev)
    out = w8_embed(ids, t, scale=2.0)
    deq = O.dequantize(*_mlx_np(q, s, b))
    ref = O.bf16_round(O.bf16_round(deq[ids.cpu().numpy()].astype(np.float32)) * 2.0)
    assert np.array_equal(out.float().cpu().numpy(), ref)
