"""GPU parity: W8 quantizer and repack (bit-exact vs oracle), activation pack (residual sum,
tap copy, RMSNorm, packed layout), skinny GEMM with its store / partial / residual / soft-cap /
gated epilogues (vs the float64 oracle), embedding gather."""

import numpy as np
import pytest
import torch

from oracle import w8 as O

pytestmark = pytest.mark.gpu


def _bf16_vals(x: torch.Tensor) -> np.ndarray:
    return x.float().cpu().numpy()


def _mlx_np(q, s, b):
    return (q.cpu().numpy(), s.view(torch.int16).cpu().numpy().view(np.uint16),
            b.view(torch.int16).cpu().numpy().view(np.uint16))


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


def test_repack_layout(dev):
    """wt[t][g][lane][16 B] and sb[t][g][16] hold exactly the MLX bytes, plain and paired."""
    from mlx_dspark.ops import W8Weight
    N, K = 64, 256
    g = torch.Generator().manual_seed(1)
    q, s, b = W8Weight.quantize_mlx((torch.randn(N, K, generator=g) * 0.02).to(dev))
    qn, sn, bn = _mlx_np(q, s, b)
    for paired in (False, True):
        W = W8Weight.from_mlx(q, s, b, paired)
        wt = W.wt.cpu().numpy().reshape(N // 16, K // 64, 64, 16)
        sb = W.sb.cpu().numpy().view(np.uint32).reshape(N // 16, K // 64, 16)
        for t in range(N // 16):
            for r in range(16):
                n = (t % 2) * (N // 2) + (t // 2) * 16 + r if paired else 16 * t + r
                for gg in range(K // 64):
                    for c in range(4):
                        assert np.array_equal(wt[t, gg, 16 * c + r], qn[n, 64 * gg + 16 * c: 64 * gg + 16 * c + 16])
                    assert sb[t, gg, r] == (int(sn[n, gg]) | (int(bn[n, gg]) << 16))


def test_pack_layout_and_unpack(dev):
    from mlx_dspark.ops import pack
    g = torch.Generator().manual_seed(3)
    for M, K in [(1, 64), (16, 4096), (17, 256), (40, 1024)]:
        x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
        p = pack(x)
        assert torch.equal(p.unpack(), x)
        # element (m, k) at P[m/16][k/64][m%16 + 16*((k%64)/16)][k%16]
        m, k = M - 1, K - 1
        G = K // 64
        idx = ((((m >> 4) * G + (k >> 6)) * 64 + (m & 15) + 16 * ((k >> 4) & 3)) << 4) + (k & 15)
        assert p.data[idx] == x[m, k]


@pytest.mark.parametrize("M,K,S", [(1, 1024, 0), (16, 4096, 4), (5, 12288, 2), (3, 3840, 1), (64, 256, 3),
                                   (16, 20480, 0)])
def test_act_pack_residual_norm(dev, M, K, S):
    from mlx_dspark.ops import act_pack
    g = torch.Generator().manual_seed(M + K + S)
    h0 = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    part = torch.randn(S, M, K, generator=g) if S else None
    h = h0.to(dev).clone()
    copy = torch.empty(M, K + 64, dtype=torch.bfloat16, device=dev)[:, 64:]
    x = act_pack(M=M, K=K, part=None if part is None else part.to(dev), h=h, copy=copy, norm_w=w.to(dev), eps=1e-6)
    # residual sum in split order, rounded once
    v = h0.float().numpy().astype(np.float32)
    if S:
        acc = np.zeros((M, K), np.float32)
        for s_ in range(S):
            acc = acc + part[s_].numpy()
        v = O.bf16_round(v + acc)
        assert np.array_equal(h.float().cpu().numpy(), v)
    assert np.array_equal(copy.float().cpu().numpy(), v)
    vf = v.astype(np.float64)
    r = 1.0 / np.sqrt((vf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    ref = O.bf16_round(((vf * r) * w.float().numpy()).astype(np.float32))
    got = x.unpack().float().cpu().numpy()
    # equal up to one bf16 ulp (the fp32 rsqrt differs from the float64 one in the last bits)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)


@pytest.mark.parametrize("M,K,S", [(16, 3840, 2), (9, 512, 8), (1, 4096, 1)])
def test_act_pack_sandwich_norm(dev, M, K, S):
    """part_norm_w: the partial sum (rounded to bf16) is RMSNorm-ed before the residual add."""
    from mlx_dspark.ops import act_pack
    g = torch.Generator().manual_seed(M * 3 + K + S)
    h0 = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
    w1 = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    w2 = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    part = torch.randn(S, M, K, generator=g)
    h = h0.to(dev).clone()
    x = act_pack(M=M, K=K, part=part.to(dev), h=h, norm_w=w2.to(dev), eps=1e-6, part_norm_w=w1.to(dev))
    acc = np.zeros((M, K), np.float32)
    for s_ in range(S):
        acc = acc + part[s_].numpy()
    ob = O.bf16_round(acc).astype(np.float64)
    r1 = 1.0 / np.sqrt((ob ** 2).mean(axis=1, keepdims=True) + 1e-6)
    n1 = O.bf16_round(((ob * r1) * w1.float().numpy()).astype(np.float32))
    v = O.bf16_round(h0.float().numpy() + n1)
    got_h = h.float().cpu().numpy()
    # one bf16 ulp of the normed term (fp32 vs float64 rsqrt) may move the sum by one ulp
    assert np.all(np.abs(got_h - v) <= np.abs(v) * 2.0 ** -7 + np.abs(n1) * 2.0 ** -7 + 1e-30)
    vf = got_h.astype(np.float64)
    r2 = 1.0 / np.sqrt((vf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    ref = O.bf16_round(((vf * r2) * w2.float().numpy()).astype(np.float32))
    got = x.unpack().float().cpu().numpy()
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (9, 256, 1024), (16, 6144, 4096), (17, 512, 4096),
                                   (36, 4096, 1024), (64, 128, 3072), (16, 192, 4096), (16, 4096, 12288),
                                   (9, 151936 // 8, 1024), (16, 1024, 3072), (3, 2048, 256), (64, 4096, 4096),
                                   (16, 151936, 4096), (16, 4096, 20480), (16, 2560, 9728), (16, 512, 2304),
                                   (4, 1024, 16640)])
def test_gemm_matches_oracle(dev, M, N, K):
    from mlx_dspark.ops import DSK_EPI_PARTIAL, W8Weight, pack, w8_gemm
    print(f"gemm M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    x = (torch.randn(M, K, generator=g) * 3.0).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    W = W8Weight.from_mlx(q, s, b)
    xp = pack(x.to(dev))
    y = w8_gemm(xp, W, out_dtype=torch.float32)
    yp = w8_gemm(xp, W, epi=DSK_EPI_PARTIAL)
    torch.cuda.synchronize()
    ref = O.gemm(_bf16_vals(x), *_mlx_np(q, s, b))
    scale = np.sqrt((ref ** 2).mean())
    err = np.abs(y.cpu().numpy() - ref).max() / scale
    assert err < 2e-4, err
    errp = np.abs(yp.sum(0).cpu().numpy() - ref).max() / scale
    assert errp < 2e-4, (errp, yp.shape)


def test_gemm_residual_softcap(dev):
    from mlx_dspark.ops import W8Weight, pack, w8_gemm
    g = torch.Generator().manual_seed(5)
    M, N, K = 16, 1024, 2048
    w = torch.randn(N, K, generator=g) * 0.02
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    W = W8Weight.from_mlx(q, s, b)
    deq = O.dequantize(*_mlx_np(q, s, b))
    big = (torch.randn(M, K + 512, generator=g) * 2).to(torch.bfloat16).to(dev)
    x = big[:, 256:256 + K]                                # strided rows, 16-byte aligned
    res = (torch.randn(M, N, generator=g)).to(torch.bfloat16)
    yd = res.to(dev).clone()
    w8_gemm(pack(x), W, out=yd, residual=yd, softcap=30.0)
    xf = x.float().cpu().numpy().astype(np.float64)
    ref = np.tanh((res.float().numpy() + xf @ deq.T) / 30.0) * 30.0
    got = yd.float().cpu().numpy()
    assert np.abs(got - ref).max() < 0.02 + 0.01 * np.abs(ref).max()


@pytest.mark.parametrize("M,I,K,act", [(16, 12288, 4096, "silu"), (9, 3072, 1024, "silu"), (40, 512, 1024, "silu"),
                                       (8, 15360 // 4, 3840, "gelu"), (2, 128, 256, "silu"), (5, 15360, 3840, "gelu")])
def test_gemm_gated_epilogue(dev, M, I, K, act):
    from mlx_dspark.ops import DSK_EPI_GEGLU, DSK_EPI_SWIGLU, W8Weight, pack, w8_gemm
    print(f"gated M={M} I={I} K={K} {act}", flush=True)
    g = torch.Generator().manual_seed(M + I + K)
    w = torch.randn(2 * I, K, generator=g) * 0.02
    x = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx(w.to(dev))
    W = W8Weight.from_mlx(q, s, b, paired=True)
    out = w8_gemm(pack(x.to(dev)), W, epi=DSK_EPI_SWIGLU if act == "silu" else DSK_EPI_GEGLU)
    got = out.unpack().float().cpu().numpy()
    gu = O.bf16_round((_bf16_vals(x).astype(np.float64) @ O.dequantize(*_mlx_np(q, s, b)).T).astype(np.float32))
    gg, uu = gu[:, :I].astype(np.float64), gu[:, I:].astype(np.float64)
    if act == "silu":
        a = gg / (1 + np.exp(-gg))
    else:
        a = 0.5 * gg * (1 + np.tanh(0.7978845608028654 * (gg + 0.044715 * gg ** 3)))
    ref = O.bf16_round((O.bf16_round(a.astype(np.float32)).astype(np.float64) * uu).astype(np.float32))
    # the projections round to bf16 before the activation: a one-ulp flip there moves the
    # product by about one ulp of the result
    err = np.abs(got - ref)
    tol = 2.0 ** -6 * np.abs(ref) + 1e-3 * np.abs(ref).max()
    assert np.mean(err <= tol) > 0.999 and err.max() < 0.05 * np.abs(ref).max(), err.max()


def test_gemm_rejects_bad_shapes(dev):
    from mlx_dspark import _hip
    from mlx_dspark.ops import W8Weight, pack, w8_gemm
    W = W8Weight.quantize(torch.randn(64, 320, device=dev) * 0.02)      # K % 256 != 0
    with pytest.raises(_hip.HipError, match="K % 256"):
        w8_gemm(pack(torch.randn(4, 320, device=dev).to(torch.bfloat16)), W)


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


# ---------------------------------------------------------------------------- 4-bit codes
def test_w4_quantize_bitexact(dev):
    from mlx_dspark.ops import W8Weight
    g = torch.Generator().manual_seed(40)
    w = torch.randn(96, 512, generator=g) * 0.02
    w[5, 0:64] = -0.5                                     # constant group
    q, s, b = W8Weight.quantize_mlx(w.to(dev), bits=4)
    qo, so, bo = O.quantize(w.numpy(), bits=4)
    assert int(q.max()) <= 15
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.view(torch.int16).cpu().numpy().view(np.uint16), so)
    assert np.array_equal(b.view(torch.int16).cpu().numpy().view(np.uint16), bo)
    # round trip within half a step (closed form)
    deq = O.dequantize(qo, so, bo)
    step = O.bits_to_f32(so).astype(np.float64)
    err = np.abs(deq - w.numpy()).reshape(96, 8, 64).max(axis=2)
    assert np.all(err <= step * 0.5 + np.abs(O.bits_to_f32(bo)) * 2 ** -8 + 1e-7)


def test_w4_repack_layout(dev):
    """wt4[t][g][lane][8 B]: byte j of a lane = codes of columns 2j (low nibble) and 2j+1 of
    its 16-column chunk, plain and paired; sb as for 8-bit."""
    from mlx_dspark.ops import W8Weight
    N, K = 64, 256
    g = torch.Generator().manual_seed(41)
    q, s, b = W8Weight.quantize_mlx((torch.randn(N, K, generator=g) * 0.02).to(dev), bits=4)
    qn, sn, bn = _mlx_np(q, s, b)
    for paired in (False, True):
        W = W8Weight.from_mlx(q, s, b, paired, bits=4)
        assert W.wt.numel() == N * K // 2 and W.nbytes == N * K // 2 + N * K // 64 * 4
        wt = W.wt.cpu().numpy().reshape(N // 16, K // 64, 64, 8)
        sb = W.sb.cpu().numpy().view(np.uint32).reshape(N // 16, K // 64, 16)
        for t in range(N // 16):
            for r in range(16):
                n = (t % 2) * (N // 2) + (t // 2) * 16 + r if paired else 16 * t + r
                for gg in range(K // 64):
                    for c in range(4):
                        codes = qn[n, 64 * gg + 16 * c: 64 * gg + 16 * c + 16]
                        assert np.array_equal(wt[t, gg, 16 * c + r], codes[0::2] | (codes[1::2] << 4))
                    assert sb[t, gg, r] == (int(sn[n, gg]) | (int(bn[n, gg]) << 16))


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (9, 256, 1024), (16, 6144, 4096), (17, 512, 4096),
                                   (64, 128, 3072), (16, 4096, 12288), (16, 151936 // 8, 1024), (16, 24576, 4096),
                                   (16, 2560, 9728), (16, 512, 2304), (16, 151936, 4096)])
def test_w4_gemm_matches_oracle(dev, M, N, K):
    from mlx_dspark.ops import DSK_EPI_PARTIAL, W8Weight, pack, w8_gemm
    print(f"w4 gemm M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 11 + N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    x = (torch.randn(M, K, generator=g) * 3.0).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx(w.to(dev), bits=4)
    W = W8Weight.from_mlx(q, s, b, bits=4)
    xp = pack(x.to(dev))
    y = w8_gemm(xp, W, out_dtype=torch.float32)
    yp = w8_gemm(xp, W, epi=DSK_EPI_PARTIAL)
    torch.cuda.synchronize()
    ref = O.gemm(_bf16_vals(x), *_mlx_np(q, s, b))
    scale = np.sqrt((ref ** 2).mean())
    err = np.abs(y.cpu().numpy() - ref).max() / scale
    assert err < 2e-4, err
    errp = np.abs(yp.sum(0).cpu().numpy() - ref).max() / scale
    assert errp < 2e-4, errp
    # a row view of the 4-bit layout multiplies like the full weight's rows
    if N >= 64 and N % 32 == 0:
        sub = W.rows(16, 48)
        ys = w8_gemm(xp, sub, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.allclose(ys, y[:, 16:48], rtol=0, atol=float(scale) * 1e-5)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_w4_gated_epilogue(dev, act):
    from mlx_dspark.ops import DSK_EPI_GEGLU, DSK_EPI_SWIGLU, W8Weight, pack, w8_gemm
    M, I, K = 7, 1024, 2048
    g = torch.Generator().manual_seed(len(act))
    wg = torch.randn(I, K, generator=g) * 0.03
    wu = torch.randn(I, K, generator=g) * 0.03
    x = (torch.randn(M, K, generator=g) * 2.0).to(torch.bfloat16)
    q, s, b = W8Weight.quantize_mlx(torch.cat([wg, wu]).to(dev), bits=4)
    W = W8Weight.from_mlx(q, s, b, paired=True, bits=4)
    out = w8_gemm(pack(x.to(dev)), W, epi=DSK_EPI_SWIGLU if act == "silu" else DSK_EPI_GEGLU)
    torch.cuda.synchronize()
    gu = O.gemm(_bf16_vals(x), *_mlx_np(q, s, b))
    gt = torch.from_numpy(gu[:, :I]).float().to(torch.bfloat16).float()
    ut = torch.from_numpy(gu[:, I:]).float().to(torch.bfloat16).float()
    if act == "silu":
        a = (gt * torch.sigmoid(gt)).to(torch.bfloat16).float()
    else:
        a = (0.5 * gt * (1 + torch.tanh(0.7978845608028654 * (gt + 0.044715 * gt ** 3)))).to(torch.bfloat16).float()
    ref = (a * ut).to(torch.bfloat16).float()
    got = out.unpack().float().cpu()
    assert (got - ref).abs().max() <= 2 ** -6 * ref.abs().max()
