"""GPU parity of the normed-later activations: dsk_act_pack_rn (residual add, bf16(h * w)
packed, per-16-column sums of h^2), the GEMM's residual epilogue (DSK_EPI_RESIDUAL: the
residual add after o_proj / down_proj inside the GEMM), and GEMMs whose x is normed later (the
RMSNorm's row scale applied to the product), against float64 closed forms and bit for bit
against each other where their arithmetic is the same; the GEMM under explicit plans
(dsk_w8_gemm_rn_planned) to the same bounds, and its rejection of plans it cannot run."""

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


def _planned(x, W, epi, y, y_dtype, ldy, plan, h=None, copy=None, next_norm=None, ssq_out=None):
    from mlx_dspark import _hip
    from mlx_dspark._hip import ptr, stream_ptr
    nt, u, waves, sk, pf = plan
    _hip.call("dsk_w8_gemm_rn_planned", ptr(x.data), ptr(W.wt), ptr(W.sb), W.bits, x.M, W.N, W.K, epi, ptr(y),
              y_dtype, ldy, 0.0, ptr(x.ssq), 0 if x.ssq is None else W.K // 16, float(x.eps), ptr(h),
              0 if h is None else h.stride(0), ptr(copy), 0 if copy is None else copy.stride(0), ptr(next_norm),
              ptr(ssq_out), nt, u, waves, sk, pf, stream_ptr())


# (slab_tiles, batch_groups, waves, k_splits, pipelined) per row-tile count: plans the planner does
# not pick for these shapes, including an empty trailing K split (5 splits of 16 four-group
# batches) and more waves than batches
_PLANS = {
    16: {"store": [(1, 2, 4, 1, 0), (2, 2, 16, 1, 1), (4, 2, 8, 1, 1), (8, 2, 4, 1, 0), (4, 4, 8, 1, 0),
                   (6, 2, 4, 1, 0), (3, 2, 8, 1, 0), (1, 4, 16, 1, 1)],
         "partial": [(2, 2, 8, 3, 0), (1, 4, 4, 5, 1), (4, 2, 16, 8, 0)],
         "gated": [(2, 2, 8, 1, 0), (4, 2, 4, 1, 0), (2, 4, 16, 1, 1)],
         "residual": [(1, 2, 16, 1, 0), (2, 2, 8, 1, 0), (1, 4, 4, 1, 0)]},
    36: {"store": [(1, 2, 16, 1, 0), (2, 2, 8, 1, 0), (4, 2, 4, 1, 0), (1, 4, 8, 1, 0)],
         "partial": [(2, 2, 4, 3, 0), (1, 2, 16, 2, 0)],
         "gated": [(2, 2, 8, 1, 0), (4, 2, 4, 1, 0)],
         "residual": [(1, 2, 8, 1, 0), (2, 2, 4, 1, 0), (1, 4, 16, 1, 0)]},
}


@pytest.mark.parametrize("M", [16, 36])
def test_planned_gemm_matches_closed_forms(dev, M):
    """dsk_w8_gemm_rn_planned under plans other than the planner's: every epilogue family (a
    normed-later x for the stores, partial sums and gated products; a plain x for the residual
    add) within the same bounds of the float64 product as the planned entry, and the partial
    slices of each plan summing to it, empty trailing slices holding zeros."""
    from mlx_dspark._hip import DSK_BF16, DSK_EPI_PARTIAL, DSK_EPI_RESIDUAL, DSK_EPI_STORE, DSK_EPI_SWIGLU, DSK_F32
    from mlx_dspark.ops import Packed, W8Weight, pack, pack_rn
    K, N, I, eps = 4096, 1536, 768, 1e-6
    g = torch.Generator().manual_seed(200 + M)
    h = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(K, generator=g)).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx((torch.randn(N, K, generator=g) * 0.02).to(dev))
    Wt = W8Weight.from_mlx(q, s, b)
    qg, sg, bg = W8Weight.quantize_mlx((torch.randn(2 * I, K, generator=g) * 0.02).to(dev))
    Wg = W8Weight.from_mlx(qg, sg, bg, paired=True)
    x = pack_rn(M=M, K=K, h=h.to(dev).clone(), norm_w=w.to(dev), eps=eps)
    hf = h.float().numpy().astype(np.float64)
    xg = _bf(hf * w.float().numpy())
    r = 1.0 / np.sqrt((hf ** 2).mean(1, keepdims=True) + eps)
    ref = r * O.gemm(xg, *_mlx_np(q, s, b))
    scale = np.sqrt((ref ** 2).mean())
    for plan in _PLANS[M]["store"]:
        print(f"planned store M={M} plan={plan}", flush=True)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
        _planned(x, Wt, DSK_EPI_STORE, y, DSK_F32, N, plan)
        torch.cuda.synchronize()
        assert np.abs(y.cpu().numpy() - ref).max() / scale < 2e-4, plan
    for plan in _PLANS[M]["partial"]:
        print(f"planned partial M={M} plan={plan}", flush=True)
        nt, u, _, sk, _ = plan
        y = torch.full((sk, M, N), float("nan"), dtype=torch.float32, device=dev)
        _planned(x, Wt, DSK_EPI_PARTIAL, y, DSK_F32, 0, plan)
        torch.cuda.synchronize()
        yc = y.cpu().numpy()
        assert np.abs(yc.sum(0) - ref).max() / scale < 2e-4, plan
        gpb = -(-(K // 64 // u) // sk) * u
        for k in range(sk):
            if k * gpb >= K // 64:
                assert not yc[k].any(), (plan, k)
    gu = r * O.gemm(xg, *_mlx_np(qg, sg, bg))
    gt, ut = _bf(gu[:, :I]).astype(np.float64), _bf(gu[:, I:]).astype(np.float64)
    ref_act = _bf(_bf(gt / (1 + np.exp(-gt))).astype(np.float64) * ut)
    for plan in _PLANS[M]["gated"]:
        print(f"planned gated M={M} plan={plan}", flush=True)
        out = Packed.empty(M, I, dev)
        _planned(x, Wg, DSK_EPI_SWIGLU, out.data, DSK_BF16, 0, plan)
        torch.cuda.synchronize()
        err = np.abs(out.unpack().float().cpu().numpy() - ref_act)
        tol = 2.0 ** -6 * np.abs(ref_act) + 1e-3 * np.abs(ref_act).max()
        assert np.mean(err <= tol) > 0.999 and err.max() < 0.05 * np.abs(ref_act).max(), (plan, err.max())
    xr = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    h0 = (torch.randn(M, N, generator=g) * 4).to(torch.bfloat16)
    wn = (1 + 0.2 * torch.randn(N, generator=g)).to(torch.bfloat16)
    rref = O.gemm(xr.float().numpy(), *_mlx_np(q, s, b))
    want = h0.float().numpy().astype(np.float64) + rref
    xp = pack(xr.to(dev))
    for plan in _PLANS[M]["residual"]:
        print(f"planned residual M={M} plan={plan}", flush=True)
        hd = h0.to(dev).clone()
        copy = torch.empty(M, 2 * N, dtype=torch.bfloat16, device=dev)[:, N:]
        yr = Packed.empty(M, N, dev, normed_later=True, eps=1e-5)
        _planned(xp, Wt, DSK_EPI_RESIDUAL, yr.data, DSK_BF16, 0, plan, h=hd, copy=copy, next_norm=wn.to(dev),
                 ssq_out=yr.ssq)
        torch.cuda.synchronize()
        got = hd.float().cpu().numpy()
        ulp = np.maximum(np.abs(want), 2.0 ** -100) * 2.0 ** -7
        assert np.all(np.abs(got - want) <= ulp + 1e-3 * np.abs(rref).max()), (plan, np.abs(got - want).max())
        assert np.array_equal(copy.float().cpu().numpy(), got), plan
        assert np.array_equal(yr.unpack().float().cpu().numpy(), _bf(got * wn.float().numpy())), plan
        assert np.array_equal(yr.ssq.cpu().numpy(), _tile_ssq(got)), plan


def test_planned_gemm_rejects_bad_plans(dev):
    """Plans with no compiled kernel or outside the entry's limits fail with DSK_EINVAL and a
    message naming the limit, before any launch."""
    from mlx_dspark import _hip
    from mlx_dspark._hip import DSK_EPI_RESIDUAL, DSK_EPI_STORE, DSK_F32
    from mlx_dspark.ops import W8Weight, pack, pack_rn
    K, N = 1024, 1536
    Wt = W8Weight.quantize(torch.randn(N, K, device=dev) * 0.02)
    xh = (torch.randn(36, K, device=dev) * 2).to(torch.bfloat16)
    x36 = pack(xh)
    x16 = pack_rn(M=16, K=K, h=xh[:16].clone(), norm_w=torch.ones(K, dtype=torch.bfloat16, device=dev), eps=1e-6)
    y = torch.empty(36, N, dtype=torch.float32, device=dev)
    h = torch.zeros(36, N, dtype=torch.bfloat16, device=dev)
    cases = [(x36, DSK_EPI_STORE, (5, 2, 4, 1, 0), "do not divide"),
             (x36, DSK_EPI_STORE, (2, 3, 4, 1, 0), "batches of 3"),
             (x36, DSK_EPI_STORE, (2, 2, 2, 1, 0), "2 waves"),
             (x36, DSK_EPI_STORE, (2, 2, 4, 2, 0), "K splits"),
             (x36, DSK_EPI_STORE, (8, 2, 16, 1, 0), "64 KB"),
             (x36, DSK_EPI_STORE, (2, 2, 8, 1, 1), "no kernel"),     # pipelined loads: one row tile only
             (x36, DSK_EPI_STORE, (2, 4, 4, 1, 0), "no kernel"),     # 4-group batches: 1-tile slabs only
             (x36, DSK_EPI_RESIDUAL, (4, 2, 4, 1, 0), "no kernel"),  # the residual add: at most 2 tiles
             (x16, DSK_EPI_RESIDUAL, (1, 2, 4, 1, 0), "no kernel")]  # the residual add takes a plain x
    for xx, epi, plan, msg in cases:
        print(f"planned reject M={xx.M} epi={epi} plan={plan}", flush=True)
        with pytest.raises(_hip.HipError, match=msg):
            _planned(xx, Wt, epi, None if epi == DSK_EPI_RESIDUAL else y, DSK_F32 if epi == DSK_EPI_STORE else 1,
                     N, plan, h=h[:xx.M] if epi == DSK_EPI_RESIDUAL else None)
    torch.cuda.synchronize()
