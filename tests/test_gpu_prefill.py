"""GPU: the dense prefill (src/mlx_dspark/generate.py:613-656 prefills the prompt in 2048-row
chunks; here a long prompt runs layer by layer over all of its rows). Its kernels against closed
forms: bf16 rows of a W8 / W4 weight bit for bit, the row RMSNorm and gated activation, and the
many-query attention (W > 64: one workgroup per 128-row query block streaming its whole key
range in 64-key blocks; causal, bidirectional and sliding-window masks, ragged rows, GQA groups
of 1 to 8) against a float32 softmax over the stored K/V; then the whole prefill against the
oracle: the
last position's logits, the tapped hidden states, and a verify block decoded from the cache it
filled."""

import numpy as np
import pytest
import torch

from _parity import Twin, check_logits
from oracle import model as OM
from oracle import w8 as O

pytestmark = pytest.mark.gpu


def _mlx_np(q, s, b):
    return (q.cpu().numpy(), s.view(torch.int16).cpu().numpy().view(np.uint16),
            b.view(torch.int16).cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("N,K,bits,paired", [(64, 256, 8, False), (256, 1024, 8, True), (96, 512, 4, False),
                                             (128, 2048, 4, True)])
def test_dequant_rows_bit_exact(dev, N, K, bits, paired):
    from mlx_dspark.ops import W8Weight, w8_dequant
    g = torch.Generator().manual_seed(N + K + bits)
    q, s, b = W8Weight.quantize_mlx((torch.randn(N, K, generator=g) * 0.05).to(dev), bits)
    W = W8Weight.from_mlx(q, s, b, paired, bits)
    got = w8_dequant(W).float().cpu().numpy()
    ref = O.bf16_round(O.dequantize(*_mlx_np(q, s, b)).astype(np.float32))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("M,K", [(1, 64), (300, 1024), (2049, 4096)])
def test_rows_rmsnorm(dev, M, K):
    from mlx_dspark.ops import rows_rmsnorm
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(K, generator=g)).to(torch.bfloat16)
    y = rows_rmsnorm(x.to(dev), w.to(dev), 1e-6).float().cpu().numpy()
    xf = x.float().numpy().astype(np.float64)
    ref = xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6) * w.float().numpy()
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_rows_gated(dev, act):
    from mlx_dspark.ops import DSK_EPI_GEGLU, DSK_EPI_SWIGLU, rows_gated
    M, I = 333, 512
    g = torch.Generator().manual_seed(5)
    gu = (torch.randn(M, 2 * I, generator=g) * 2).to(torch.bfloat16)
    out = rows_gated(gu.to(dev), DSK_EPI_SWIGLU if act == "silu" else DSK_EPI_GEGLU).float().cpu()
    gt, ut = gu[:, :I].float(), gu[:, I:].float()
    a = gt * torch.sigmoid(gt) if act == "silu" else 0.5 * gt * (1 + torch.tanh(0.7978845608028654 * (gt + 0.044715 * gt ** 3)))
    ref = (a.to(torch.bfloat16).float() * ut).to(torch.bfloat16).float()
    assert (out - ref).abs().max() <= 2 ** -6 * ref.abs().max()


def _pool_rows(cache, l, n, which):
    """[n, nkv, hd] float values the cache holds for tokens 0..n-1 of row 0 (dequantized)."""
    page = cache.page
    pool = cache.k[l] if which == "k" else cache.v[l]
    sb = cache.k_sb[l] if which == "k" else cache.v_sb[l]
    bt = cache.block_table[0].cpu().numpy()
    rows = []
    for j in range(n):
        p = int(bt[j // page])
        if sb is None:
            rows.append(pool[p, :, j % page].float().cpu())
        else:
            q = pool[p, :, j % page].cpu().numpy().astype(np.float64)
            w = sb[p, :, j % page].cpu().numpy().view(np.uint32)
            s = O.bits_to_f32((w & 0xFFFF).astype(np.uint16)).astype(np.float64)
            bb = O.bits_to_f32((w >> 16).astype(np.uint16)).astype(np.float64)
            v = q.reshape(q.shape[0], -1, 64) * s[..., None] + bb[..., None]
            rows.append(torch.from_numpy(O.bf16_round(v.reshape(q.shape).astype(np.float32))))
    return torch.stack(rows)


@pytest.mark.parametrize("kv_bits,L0,W", [(None, 0, 300), (8, 100, 300), (8, 500, 777), (None, 64, 129)])
def test_many_query_attention(dev, kv_bits, L0, W):
    """Causal attention of W > 64 new rows over the cache: float32 softmax over the stored K/V."""
    from mlx_dspark import ops
    from mlx_dspark.kv import PagedKVCache
    print(f"many-query attention kv_bits={kv_bits} L0={L0} W={W}", flush=True)
    nq, nkv, hd = 8, 2, 128
    cache = PagedKVCache(1, 1, nkv, hd, L0 + W + 64, kv_bits=kv_bits)
    g = torch.Generator().manual_seed(L0 + W)
    qkv = (torch.randn(L0 + W, (nq + 2 * nkv) * hd, generator=g)).to(torch.bfloat16).to(dev)
    inv = ops.rope_inv_freq(hd, 1e6, dev)
    for r0, r1 in ((0, L0), (L0, L0 + W)):
        if r1 > r0:
            q = ops.qkv_rope_append(qkv[r0:r1].contiguous(), 1, r1 - r0, nq, nkv, hd, None, None, 1e-6, inv,
                                    cache.seq_lens, cache.block_table, cache.page, cache.kv_dtype, *cache.layer_args(0))
            if r0 == L0:
                out = ops.attention(q, 1, W, nq, nkv, hd, hd ** -0.5, cache.seq_lens, cache.max_ctx,
                                    cache.block_table, cache.page, cache.kv_dtype, *cache.layer_args(0))
            ops.lens_add(cache.seq_lens, None, r1 - r0)
    torch.cuda.synchronize()
    K, V = _pool_rows(cache, 0, L0 + W, "k"), _pool_rows(cache, 0, L0 + W, "v")
    qf = q.float().cpu().view(W, nq, hd)
    ref = OM.sdpa(qf, K, V, hd ** -0.5, OM.causal_mask(L0, W))
    got = out.float().cpu().view(W, nq, hd)
    err = (got - ref).abs().max() / ref.abs().max()
    assert err < 2e-2, err


@pytest.mark.parametrize("kv_bits,lens,W,nq,nkv,causal,window", [
    (8, [100, 1000], 300, 8, 2, True, 0),        # ragged rows, G = 4
    (None, [0], 1100, 4, 2, True, 0),            # 18 key blocks through both LDS buffers, G = 2
    (8, [50, 7], 130, 2, 2, False, 0),           # bidirectional, G = 1
    (8, [400], 200, 8, 2, True, 128),            # sliding window
    (None, [0, 64, 333], 65, 16, 2, True, 0),    # one row past the verify width, G = 8
])
def test_many_query_attention_masks_and_rows(dev, kv_bits, lens, W, nq, nkv, causal, window):
    """Random K/V written straight into shuffled pages (8-bit codes with random scale / bias
    words, or bf16), random queries; each row b's query i sits at position lens[b] + i."""
    from mlx_dspark import ops
    from mlx_dspark.kv import PagedKVCache
    print(f"many-query attention kv_bits={kv_bits} lens={lens} W={W} nq={nq} nkv={nkv} causal={causal} "
          f"window={window}", flush=True)
    hd, B = 128, len(lens)
    max_ctx = max(lens) + W + 64
    cache = PagedKVCache(1, B, nkv, hd, max_ctx, kv_bits=kv_bits, spare_pages=5)
    g = torch.Generator().manual_seed(sum(lens) + W + nq)
    perm = torch.randperm(cache.n_pages, generator=g)[: B * cache.max_pages]
    cache.block_table.copy_(perm.view(B, cache.max_pages).to(torch.int32))
    if kv_bits is None:
        for pool in (cache.k[0], cache.v[0]):
            pool.copy_(torch.randn(pool.shape, generator=g).to(torch.bfloat16))
    else:
        for pool, sb in ((cache.k[0], cache.k_sb[0]), (cache.v[0], cache.v_sb[0])):
            pool.copy_(torch.randint(0, 256, pool.shape, generator=g, dtype=torch.uint8))
            sc = (0.01 + 0.02 * torch.rand(sb.shape, generator=g)).to(torch.bfloat16).view(torch.int16)
            bi = (-2.0 + torch.rand(sb.shape, generator=g)).to(torch.bfloat16).view(torch.int16)
            sb.copy_((sc.int() & 0xFFFF) | (bi.int() << 16))
    cache.set_lengths(lens)
    q = torch.randn(B * W, nq * hd, generator=g).to(torch.bfloat16).to(dev)
    out = ops.attention(q, B, W, nq, nkv, hd, hd ** -0.5, cache.seq_lens, cache.max_ctx, cache.block_table,
                        cache.page, cache.kv_dtype, *cache.layer_args(0), causal=causal, window=window)
    torch.cuda.synchronize()
    got = out.float().cpu().view(B, W, nq, hd)
    G = nq // nkv
    worst = 0.0
    for b, L0 in enumerate(lens):
        n = L0 + W
        K, V = _row_pool_rows(cache, b, n, "k"), _row_pool_rows(cache, b, n, "v")   # [n, nkv, hd]
        pos = torch.arange(L0, L0 + W)[:, None]
        j = torch.arange(n)[None, :]
        allowed = j <= pos if causal else torch.ones(W, n, dtype=torch.bool)
        if window:
            allowed = allowed & (j > pos - window)
        qf = q.float().cpu().view(B, W, nq, hd)[b]
        for h in range(nq):
            sc = (qf[:, h] @ K[:, h // G].T) * hd ** -0.5
            sc = sc.masked_fill(~allowed, float("-inf"))
            ref = torch.softmax(sc, -1) @ V[:, h // G]
            worst = max(worst, float((got[b, :, h] - ref).abs().max() / ref.abs().max()))
    assert worst < 2e-2, worst


@pytest.mark.parametrize("kv_bits,lens,W,hd,window", [
    (8, [3000], 9, 256, 1024),          # split kernel, head_dim 256: splits before the window skipped
    (None, [2000, 300], 100, 256, 700), # its many-query form (query-tile groups on the grid)
    (8, [3000, 40], 16, 128, 512),      # the verify kernel with a window
])
def test_sliding_window_attention_over_long_context(dev, kv_bits, lens, W, hd, window):
    """Causal sliding-window attention where most of a row's context lies before its window:
    the output against a float32 softmax over the window's keys."""
    from mlx_dspark import ops
    from mlx_dspark.kv import PagedKVCache
    print(f"window attention kv_bits={kv_bits} lens={lens} W={W} hd={hd} window={window}", flush=True)
    nq, nkv, B = 4, 2, len(lens)
    cache = PagedKVCache(1, B, nkv, hd, max(lens) + W + 64, kv_bits=kv_bits, spare_pages=3)
    g = torch.Generator().manual_seed(sum(lens) + hd + window)
    perm = torch.randperm(cache.n_pages, generator=g)[: B * cache.max_pages]
    cache.block_table.copy_(perm.view(B, cache.max_pages).to(torch.int32))
    if kv_bits is None:
        for pool in (cache.k[0], cache.v[0]):
            pool.copy_(torch.randn(pool.shape, generator=g).to(torch.bfloat16))
    else:
        for pool, sb in ((cache.k[0], cache.k_sb[0]), (cache.v[0], cache.v_sb[0])):
            pool.copy_(torch.randint(0, 256, pool.shape, generator=g, dtype=torch.uint8))
            sc = (0.01 + 0.02 * torch.rand(sb.shape, generator=g)).to(torch.bfloat16).view(torch.int16)
            bi = (-2.0 + torch.rand(sb.shape, generator=g)).to(torch.bfloat16).view(torch.int16)
            sb.copy_((sc.int() & 0xFFFF) | (bi.int() << 16))
    cache.set_lengths(lens)
    q = torch.randn(B * W, nq * hd, generator=g).to(torch.bfloat16).to(dev)
    out = ops.attention(q, B, W, nq, nkv, hd, hd ** -0.5, cache.seq_lens, cache.max_ctx, cache.block_table,
                        cache.page, cache.kv_dtype, *cache.layer_args(0), causal=True, window=window)
    torch.cuda.synchronize()
    got = out.float().cpu().view(B, W, nq, hd)
    G = nq // nkv
    worst = 0.0
    for b, L0 in enumerate(lens):
        n = L0 + W
        K, V = _row_pool_rows(cache, b, n, "k"), _row_pool_rows(cache, b, n, "v")
        pos = torch.arange(L0, L0 + W)[:, None]
        j = torch.arange(n)[None, :]
        allowed = (j <= pos) & (j > pos - window)
        qf = q.float().cpu().view(B, W, nq, hd)[b]
        for h in range(nq):
            sc = ((qf[:, h] @ K[:, h // G].T) * hd ** -0.5).masked_fill(~allowed, float("-inf"))
            ref = torch.softmax(sc, -1) @ V[:, h // G]
            worst = max(worst, float((got[b, :, h] - ref).abs().max() / ref.abs().max()))
    assert worst < 2e-2, worst


def _row_pool_rows(cache, b, n, which):
    """[n, nkv, hd] float values of row b's tokens 0..n-1 (dequantized as the kernels do)."""
    page = cache.page
    pool = (cache.k if which == "k" else cache.v)[0].cpu()
    sb = (cache.k_sb if which == "k" else cache.v_sb)[0]
    sb = None if sb is None else sb.cpu().numpy().view(np.uint32)
    bt = cache.block_table[b].cpu().numpy()
    rows = []
    for j in range(n):
        p = int(bt[j // page])
        if sb is None:
            rows.append(pool[p, :, j % page].float())
        else:
            qv = pool[p, :, j % page].numpy().astype(np.float32)
            w = sb[p, :, j % page]
            sc = O.bits_to_f32((w & 0xFFFF).astype(np.uint16))
            bi = O.bits_to_f32((w >> 16).astype(np.uint16))
            v = qv.reshape(qv.shape[0], -1, 64) * sc[..., None] + bi[..., None]
            rows.append(torch.from_numpy(O.bf16_round(v.reshape(qv.shape).astype(np.float32))))
    return torch.stack(rows)


def test_dense_prefill_matches_oracle(dev):
    from mlx_dspark import synthetic
    print("dense prefill vs oracle: tiny model, 700-token prompt, taps 1 and 3, then a 9-row verify", flush=True)
    model = synthetic.build_target("tiny", seed=21, keep_mlx=True)
    synthetic.randomize_norms(model, seed=22)
    V = model.args.vocab_size
    prompt = np.random.default_rng(3).integers(0, V, 700).tolist()
    block = np.random.default_rng(4).integers(0, V, 9).tolist()
    cache = model.make_cache(max_ctx=800)
    logits, fused = model.prefill(prompt, cache, [1, 3])
    assert cache.lengths[0] == 700 and int(cache.seq_lens[0]) == 700
    vl, _ = model.forward(torch.tensor([block], dtype=torch.int32, device=dev), cache, None)
    torch.cuda.synchronize()
    ref = Twin(lambda: OM.OracleTarget(model))
    ref.dense = True                     # the prompt with the dense prefill's rounding
    (rl, rf), (el, _) = ref.forward(prompt, tap=(1, 3))
    ref.dense = False
    check_logits(logits[0, -1].float().cpu(), rl[-1], "dense prefill, last position", exact=el[-1])
    tap_err = float((fused[0].float().cpu() - rf).abs().max() / rf.abs().max())
    assert tap_err < 2e-2, tap_err
    (rvl, _), (evl, _) = ref.forward(block)
    check_logits(vl[0].float().cpu(), rvl, "verify rows over the dense-prefilled cache", exact=evl)
    # the chunked forward passes (the verify's rounding) fill an equivalent cache
    c2 = model.make_cache(max_ctx=800)
    l2, _ = model.prefill(prompt, c2, None, dense=False)
    torch.cuda.synchronize()
    (cl, _), (ecl, _) = Twin(lambda: OM.OracleTarget(model)).forward(prompt)
    check_logits(l2[0, -1].float().cpu(), cl[-1], "chunked prefill, last position", exact=ecl[-1])


def test_dense_prefill_with_held_weights_is_bit_identical(dev):
    """keep_dense_weights: the prefill over the held bf16 rows writes the same cache, taps and
    logits, bit for bit, as the prefill that expands each layer's weights as it goes."""
    from mlx_dspark import synthetic
    print("dense prefill: held bf16 weight rows against per-layer expansion, tiny model, 600 tokens", flush=True)
    model = synthetic.build_target("tiny", seed=31)
    prompt = np.random.default_rng(5).integers(0, model.args.vocab_size, 600).tolist()
    outs = []
    for keep in (False, True):
        held = model.keep_dense_weights(keep)
        assert (held > 0) == keep
        cache = model.make_cache(max_ctx=700)
        logits, fused = model.prefill(prompt, cache, [0, 2])
        torch.cuda.synchronize()
        outs.append((logits.clone(), fused.clone(), [k.clone() for k in cache.k], [v.clone() for v in cache.v]))
    model.keep_dense_weights(False)
    (la, fa, ka, va), (lb, fb, kb, vb) = outs
    assert torch.equal(la, lb) and torch.equal(fa, fb)
    assert all(torch.equal(x, y) for x, y in zip(ka, kb)) and all(torch.equal(x, y) for x, y in zip(va, vb))
