"""GPU parity of the normed-later activations: dsk_act_pack_rn (residual add, bf16(h * w)
packed, per-16-column sums of h^2), the GEMM's residual epilogue (DSK_EPI_RESIDUAL: the
residual add after o_proj / down_proj inside the GEMM), and GEMMs whose x is normed later (the
RMSNorm's row scale applied to the product), against float64 closed forms and bit for bit
against each other where their arithmetic is the same."""

import numpy as np
import pytest
import torch

from oracle import w8 as O

pytestmark = pytest.mark.gpu


def _bf(x: np.ndarray) -> np.ndarray:
    return O.bf16_round(np.asarray(x, dtype=np.float32))


def _tile_ssq(hn: np.ndarray) -> np.ndarray:
    """[M, K/16] float32 sums of squares per 16-column tile, as the balanced tree
    ((h0^2 + h1^2) + (h2^2 + h3^2)) + ... that both kernels use."""
    M, K = hn.shape
    v = (hn.astype(np.float32) * hn.astype(np.float32)).reshape(M, K // 16, 16)
    while v.shape[-1] > 1:
        v = (v[..., 0::2] + v[..., 1::2]).astype(np.float32)
    return np.ascontiguousarray(v[..., 0])


def _mlx_np(q, s, b):
    return (q.cpu().numpy(), s.view(torch.int16).cpu().numpy().view(np.uint16),
            b.view(torch.int16).cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("M,K,S", [(1, 1024, 0), (16, 4096, 0), (16, 4096, 8), (9, 1024, 2), (64, 4096, 4),
                                   (36, 3840, 1)])
def test_pack_rn_closed_form(dev, M, K, S):
    from mlx_dspark.ops import pack_rn
    print(f"pack_rn M={M} K={K} S={S}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + K + S)
    h0 = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(K, generator=g)).to(torch.bfloat16)
    part = torch.randn(S, M, K, generator=g) if S else None
    h = h0.to(dev).clone()
    copy = torch.empty(M, K + 64, dtype=torch.bfloat16, device=dev)[:, 64:]
    x = pack_rn(M=M, K=K, h=h, norm_w=w.to(dev), eps=1e-6, part=None if part is None else part.to(dev), copy=copy)
    torch.cuda.synchronize()
    if S:
        acc = np.zeros((M, K), np.float32)
        for s in range(S):
            acc = (acc + part[s].numpy()).astype(np.float32)
        hn = _bf(h0.float().numpy() + acc)
    else:
        hn = h0.float().numpy()
    assert np.array_equal(h.float().cpu().numpy(), hn)
    if S:
        assert np.array_equal(copy.float().cpu().numpy(), hn)
    assert np.array_equal(x.unpack().float().cpu().numpy(), _bf(hn * w.float().numpy()))
    assert np.array_equal(x.ssq.cpu().numpy(), _tile_ssq(hn))
    r = x.row_scale().cpu().numpy()
    r_ref = 1.0 / np.sqrt((hn.astype(np.float64) ** 2).mean(1) + 1e-6)
    assert np.allclose(r, r_ref, rtol=1e-5)


@pytest.mark.parametrize("M,N,K,bits", [(1, 1024, 2048, 8), (16, 4096, 4096, 8), (16, 4096, 12288, 8),
                                        (9, 1024, 3072, 8), (17, 2048, 1024, 8), (36, 4096, 4096, 8),
                                        (64, 4096, 12288, 8), (16, 4096, 4096, 4)])
def test_residual_epilogue(dev, M, N, K, bits):
    """h += x . W^T in the GEMM epilogue: h within one rounding of the float64 product added to
    h0, and the tap copy, bf16(h * w) and the tile sums exact functions of the h it wrote."""
    from mlx_dspark.ops import W8Weight, pack, w8_residual
    print(f"residual epilogue M={M} N={N} K={K} bits={bits}", flush=True)
    g = torch.Generator().manual_seed(M + N + K + bits)
    W8 = torch.randn(N, K, generator=g) * 0.02
    x = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    h0 = (torch.randn(M, N, generator=g) * 4).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(N, generator=g)).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx(W8.to(dev), bits=bits)
    Wt = W8Weight.from_mlx(q, s, b, bits=bits)
    h = h0.to(dev).clone()
    copy = torch.empty(M, 2 * N, dtype=torch.bfloat16, device=dev)[:, N:]
    y = w8_residual(pack(x.to(dev)), Wt, h, next_norm=w.to(dev), eps=1e-5, copy=copy)
    torch.cuda.synchronize()
    ref = O.gemm(x.float().numpy(), *_mlx_np(q, s, b))
    want = h0.float().numpy().astype(np.float64) + ref
    got = h.float().cpu().numpy()
    ulp = np.maximum(np.abs(want), 2.0 ** -100) * 2.0 ** -7
    assert np.all(np.abs(got - want) <= ulp + 1e-3 * np.abs(ref).max()), np.abs(got - want).max()
    assert np.array_equal(copy.float().cpu().numpy(), got)
    assert np.array_equal(y.unpack().float().cpu().numpy(), _bf(got * w.float().numpy()))
    assert np.array_equal(y.ssq.cpu().numpy(), _tile_ssq(got))
    # without an output: h and the copy only
    h2 = h0.to(dev).clone()
    assert w8_residual(pack(x.to(dev)), Wt, h2, next_norm=None, eps=1e-5, out=False) is None
    torch.cuda.synchronize()
    assert torch.equal(h2, h)


@pytest.mark.parametrize("M", [1, 9, 16, 17, 36, 64])
def test_normed_later_consumers(dev, M):
    """Every epilogue family with a normed-later x: the product of bf16(h * w) scaled by
    rsqrt(mean(h^2) + eps) per row (float64 closed form), and close to the normalise-first
    product (one bf16 rounding of the normalised x apart)."""
    from mlx_dspark.ops import DSK_EPI_PARTIAL, DSK_EPI_SWIGLU, W8Weight, pack, pack_rn, w8_gemm
    print(f"normed-later consumers M={M}", flush=True)
    K, N, I = 4096, 1024, 1024
    eps = 1e-6
    g = torch.Generator().manual_seed(100 + M)
    h = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(K, generator=g)).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx((torch.randn(N, K, generator=g) * 0.02).to(dev))
    Wt = W8Weight.from_mlx(q, s, b)
    qg, sg, bg = W8Weight.quantize_mlx((torch.randn(2 * I, K, generator=g) * 0.02).to(dev))
    Wg = W8Weight.from_mlx(qg, sg, bg, paired=True)
    hd = h.to(dev)
    x = pack_rn(M=M, K=K, h=hd.clone(), norm_w=w.to(dev), eps=eps)
    y = w8_gemm(x, Wt, out_dtype=torch.float32)
    yp = w8_gemm(x, Wt, epi=DSK_EPI_PARTIAL)
    act = w8_gemm(x, Wg, epi=DSK_EPI_SWIGLU)
    first = w8_gemm(pack(hd, w.to(dev), eps), Wt, out_dtype=torch.float32)
    torch.cuda.synchronize()
    hf = h.float().numpy().astype(np.float64)
    xg = _bf(hf * w.float().numpy())
    r = 1.0 / np.sqrt((hf ** 2).mean(1, keepdims=True) + eps)
    ref = r * O.gemm(xg, *_mlx_np(q, s, b))
    scale = np.sqrt((ref ** 2).mean())
    assert np.abs(y.cpu().numpy() - ref).max() / scale < 2e-4
    assert np.abs(yp.sum(0).cpu().numpy() - ref).max() / scale < 2e-4
    assert np.abs(first.cpu().numpy() - ref).max() / scale < 2e-2
    gu = r * O.gemm(xg, *_mlx_np(qg, sg, bg))
    gt, ut = _bf(gu[:, :I]).astype(np.float64), _bf(gu[:, I:]).astype(np.float64)
    a = _bf(gt / (1 + np.exp(-gt))).astype(np.float64)
    ref_act = _bf(a * ut)
    got = act.unpack().float().cpu().numpy()
    err = np.abs(got - ref_act)
    tol = 2.0 ** -6 * np.abs(ref_act) + 1e-3 * np.abs(ref_act).max()
    assert np.mean(err <= tol) > 0.999 and err.max() < 0.05 * np.abs(ref_act).max(), err.max()
