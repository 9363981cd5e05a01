"""GPU parity: q/k RMSNorm + RoPE + paged KV append, and split-K paged attention
(causal-with-offset and bidirectional, bf16 and 8-bit KV) against float32 references."""

import math

import numpy as np
import pytest
import torch

from oracle import w8 as O

pytestmark = pytest.mark.gpu


def _rope_ref(x, pos, inv_freq):
    # x [..., hd] float32; rotate-half
    hd = x.shape[-1]
    ang = pos[:, None].float() * inv_freq[None, :]                  # [n, hd/2]
    c, s = torch.cos(ang), torch.sin(ang)
    x1, x2 = x[..., : hd // 2], x[..., hd // 2:]
    while c.dim() < x1.dim():
        c, s = c.unsqueeze(1), s.unsqueeze(1)
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def _rms(x, w, eps):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w


class Pool:
    def __init__(self, B, nkv, hd, max_ctx, page, kv_dtype, dev, seed=0):
        self.page = page
        self.max_pages = (max_ctx + page - 1) // page
        n_pages = B * self.max_pages + 3
        g = torch.Generator().manual_seed(seed)
        perm = torch.randperm(n_pages, generator=g)[: B * self.max_pages]
        self.block_table = perm.view(B, self.max_pages).to(torch.int32).to(dev)   # shuffled pages
        shape = (n_pages, nkv, page, hd)
        if kv_dtype == 0:
            self.k = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
            self.v = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
            self.ksb = self.vsb = None
        else:
            self.k = torch.zeros(shape, dtype=torch.uint8, device=dev)
            self.v = torch.zeros(shape, dtype=torch.uint8, device=dev)
            self.ksb = torch.zeros((n_pages, nkv, page, hd // 64), dtype=torch.int32, device=dev)
            self.vsb = torch.zeros_like(self.ksb)
        self.kv_dtype = kv_dtype

    def read(self, b, n, which):
        """token-major [n, nkv, hd] float32 values as stored (dequantized for u8)."""
        bt = self.block_table[b].cpu()
        pool = self.k if which == "k" else self.v
        sb = self.ksb if which == "k" else self.vsb
        rows = []
        for j in range(n):
            p = int(bt[j // self.page])
            if self.kv_dtype == 0:
                rows.append(pool[p, :, j % self.page].float().cpu())
            else:
                q = pool[p, :, j % self.page].cpu().numpy()
                s = sb[p, :, j % self.page].cpu().numpy().view(np.uint32)
                sc = O.bits_to_f32((s & 0xFFFF).astype(np.uint16))
                bi = O.bits_to_f32((s >> 16).astype(np.uint16))
                hd = q.shape[-1]
                val = q.reshape(q.shape[0], hd // 64, 64).astype(np.float32) * sc[..., None] + bi[..., None]
                rows.append(torch.from_numpy(O.bf16_round(val.reshape(q.shape[0], hd))))
        return torch.stack(rows)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("kv_dtype", [0, 1])
@pytest.mark.parametrize("B,W,L0,causal", [(1, 16, 0, True), (1, 16, 700, True), (2, 9, 37, True),
                                           (1, 1, 300, True), (2, 8, 130, False), (1, 64, 64, True),
                                           (1, 16, 120, True), (2, 16, 250, False)])
def test_append_and_attention(dev, kv_dtype, B, W, L0, causal, fused):
    """fused=False: dsk_qkv_rope_append then dsk_attention; fused=True: dsk_qkv_attention (the
    queries are then checked through the attention output only)."""
    from mlx_dspark.ops import attention, qkv_attention, qkv_rope_append, rope_inv_freq
    print(f"attn fused={fused} kv={kv_dtype} B={B} W={W} L0={L0} causal={causal}", flush=True)
    nq, nkv, hd, page = 8, 2, 128, 64
    eps, theta = 1e-6, 1e6
    g = torch.Generator().manual_seed(B * 1000 + W * 10 + L0)
    max_ctx = L0 + W + 5
    pool = Pool(B, nkv, hd, max_ctx, page, kv_dtype, dev, seed=L0 + W)
    inv = rope_inv_freq(hd, theta, dev)
    qn = (1 + 0.1 * torch.randn(hd, generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(hd, generator=g)).to(torch.bfloat16)
    nh = nq + 2 * nkv
    zeros = torch.zeros(B, dtype=torch.int32, device=dev)
    # prefix tokens (previous rounds), then the W new tokens
    if L0:
        pre = (torch.randn(B * L0, nh * hd, generator=g)).to(torch.bfloat16).to(dev)
        qkv_rope_append(pre, B, L0, nq, nkv, hd, qn.to(dev), kn.to(dev), eps, inv, zeros, pool.block_table, page,
                        kv_dtype, pool.k, pool.v, pool.ksb, pool.vsb)
    qkv = (torch.randn(B * W, nh * hd, generator=g)).to(torch.bfloat16)
    sl = torch.full((B,), L0, dtype=torch.int32, device=dev)
    scale = hd ** -0.5
    if fused:
        q = None
        out = qkv_attention(qkv.to(dev), B, W, nq, nkv, hd, qn.to(dev), kn.to(dev), eps, inv, scale, sl, max_ctx,
                            pool.block_table, page, kv_dtype, pool.k, pool.v, pool.ksb, pool.vsb, causal=causal)
    else:
        q = qkv_rope_append(qkv.to(dev), B, W, nq, nkv, hd, qn.to(dev), kn.to(dev), eps, inv, sl,
                            pool.block_table, page, kv_dtype, pool.k, pool.v, pool.ksb, pool.vsb)
        out = attention(q, B, W, nq, nkv, hd, scale, sl, max_ctx, pool.block_table, page, kv_dtype, pool.k,
                        pool.v, pool.ksb, pool.vsb, causal=causal)
    torch.cuda.synchronize()

    # append check: q and the newly stored K/V against the float32 prologue
    invc = inv.cpu()
    x = qkv.float().view(B, W, nh, hd)
    pos = (torch.arange(W) + L0)
    qrefs = []
    for b in range(B):
        qr = _rope_ref(_rms(x[b, :, :nq], qn.float(), eps), pos, invc)
        qrefs.append(qr.to(torch.bfloat16).float())
        if q is not None:
            assert (q.view(B, W, nq, hd)[b].float().cpu() - qr).abs().max() < 0.05
        kr = _rope_ref(_rms(x[b, :, nq:nq + nkv], kn.float(), eps), pos, invc)
        vr = x[b, :, nq + nkv:]
        ks = pool.read(b, L0 + W, "k")[L0:]
        vs = pool.read(b, L0 + W, "v")[L0:]
        tol = 0.05 if kv_dtype == 0 else 0.1
        assert (ks - kr).abs().max() < tol
        assert (vs - vr).abs().max() < tol

    # attention check against the stored K/V
    G = nq // nkv
    for b in range(B):
        K = pool.read(b, L0 + W, "k")          # [Lk, nkv, hd]
        V = pool.read(b, L0 + W, "v")
        qb = qrefs[b] if q is None else q.view(B, W, nq, hd)[b].float().cpu()
        ref = torch.empty(W, nq, hd)
        for h in range(nq):
            s = (qb[:, h] @ K[:, h // G].T) * scale          # [W, Lk]
            if causal:
                j = torch.arange(L0 + W)[None, :]
                i = torch.arange(W)[:, None]
                s = s.masked_fill(j > L0 + i, float("-inf"))
            ref[:, h] = torch.softmax(s, -1) @ V[:, h // G]
        got = out.view(B, W, nq, hd)[b].float().cpu()
        err = (got - ref).abs().max().item()
        assert err < 2e-2, err


@pytest.mark.parametrize("L0", [0, 300, 4100])
def test_partial_qkv_input_and_packed_output(dev, L0):
    """Split-K partial sums as the rope input and the packed (o-projection) output layout give
    the same q, cache contents and attention output as the bf16 / row-major path."""
    from mlx_dspark.ops import attention, qkv_rope_append, rope_inv_freq
    print(f"partial/packed L0={L0}", flush=True)
    B, W, nq, nkv, hd, page = 1, 16, 8, 2, 128, 64
    g = torch.Generator().manual_seed(L0 + 7)
    max_ctx = L0 + W + 5
    nh = nq + 2 * nkv
    inv = rope_inv_freq(hd, 1e6, dev)
    qn = torch.full((hd,), hd ** -0.25).to(torch.bfloat16).to(dev)
    pools = [Pool(B, nkv, hd, max_ctx, page, 1, dev, seed=3) for _ in range(2)]
    sl = torch.full((B,), L0, dtype=torch.int32, device=dev)
    if L0:
        pre = torch.randn(B * L0, nh * hd, generator=g).to(torch.bfloat16).to(dev)
        for p in pools:
            zeros = torch.zeros(B, dtype=torch.int32, device=dev)
            for c0 in range(0, L0, 64):
                c1 = min(L0, c0 + 64)
                z = zeros + c0
                qkv_rope_append(pre[c0:c1], B, c1 - c0, nq, nkv, hd, qn, qn, 1e-6, inv, z, p.block_table, page, 1,
                                p.k, p.v, p.ksb, p.vsb)
    parts = torch.randn(3, B * W, nh * hd, generator=g).to(dev)
    summed = parts[0] + parts[1] + parts[2]
    q_a = qkv_rope_append(summed.to(torch.bfloat16), B, W, nq, nkv, hd, qn, qn, 1e-6, inv, sl, pools[0].block_table,
                          page, 1, pools[0].k, pools[0].v, pools[0].ksb, pools[0].vsb)
    q_b = qkv_rope_append(parts, B, W, nq, nkv, hd, qn, qn, 1e-6, inv, sl, pools[1].block_table, page, 1,
                          pools[1].k, pools[1].v, pools[1].ksb, pools[1].vsb)
    assert torch.equal(q_a, q_b)
    assert torch.equal(pools[0].k, pools[1].k) and torch.equal(pools[0].vsb, pools[1].vsb)
    kw = dict(causal=True)
    o_a = attention(q_a, B, W, nq, nkv, hd, hd ** -0.5, sl, max_ctx, pools[0].block_table, page, 1, pools[0].k,
                    pools[0].v, pools[0].ksb, pools[0].vsb, **kw)
    o_b = attention(q_b, B, W, nq, nkv, hd, hd ** -0.5, sl, max_ctx, pools[1].block_table, page, 1, pools[1].k,
                    pools[1].v, pools[1].ksb, pools[1].vsb, packed=True, **kw)
    assert torch.equal(o_a, o_b.unpack())


@pytest.mark.parametrize("L0", [0, 120, 4100])
def test_fused_partial_input_and_packed_output(dev, L0):
    """dsk_qkv_attention: fp32 split-K slices give bit-identical cache contents and output to
    the bf16 rounding of their sum, and the packed output equals the row-major one."""
    from mlx_dspark.ops import qkv_attention, qkv_rope_append, rope_inv_freq
    print(f"fused partial/packed L0={L0}", flush=True)
    B, W, nq, nkv, hd, page = 1, 16, 8, 2, 128, 64
    g = torch.Generator().manual_seed(L0 + 11)
    max_ctx = L0 + W + 5
    nh = nq + 2 * nkv
    inv = rope_inv_freq(hd, 1e6, dev)
    qn = torch.full((hd,), hd ** -0.25).to(torch.bfloat16).to(dev)
    pools = [Pool(B, nkv, hd, max_ctx, page, 1, dev, seed=5) for _ in range(2)]
    sl = torch.full((B,), L0, dtype=torch.int32, device=dev)
    if L0:
        pre = torch.randn(B * L0, nh * hd, generator=g).to(torch.bfloat16).to(dev)
        for p in pools:
            zeros = torch.zeros(B, dtype=torch.int32, device=dev)
            for c0 in range(0, L0, 64):
                c1 = min(L0, c0 + 64)
                qkv_rope_append(pre[c0:c1], B, c1 - c0, nq, nkv, hd, qn, qn, 1e-6, inv, zeros + c0, p.block_table,
                                page, 1, p.k, p.v, p.ksb, p.vsb)
    parts = torch.randn(3, B * W, nh * hd, generator=g).to(dev)
    summed = (parts[0] + parts[1] + parts[2]).to(torch.bfloat16)
    args = dict(causal=True)
    o_a = qkv_attention(summed, B, W, nq, nkv, hd, qn, qn, 1e-6, inv, hd ** -0.5, sl, max_ctx,
                        pools[0].block_table, page, 1, pools[0].k, pools[0].v, pools[0].ksb, pools[0].vsb, **args)
    o_b = qkv_attention(parts, B, W, nq, nkv, hd, qn, qn, 1e-6, inv, hd ** -0.5, sl, max_ctx, pools[1].block_table,
                        page, 1, pools[1].k, pools[1].v, pools[1].ksb, pools[1].vsb, packed=True, **args)
    torch.cuda.synchronize()
    assert torch.equal(pools[0].k, pools[1].k) and torch.equal(pools[0].v, pools[1].v)
    assert torch.equal(pools[0].ksb, pools[1].ksb) and torch.equal(pools[0].vsb, pools[1].vsb)
    assert torch.equal(o_a, o_b.unpack())


def _read_tokens(pool, b, n, which):
    """token-major [n, nkv, hd] float32 of row b (dequantized for u8), all pages gathered at once."""
    pages = pool.block_table[b, : (n + pool.page - 1) // pool.page].long()
    data = (pool.k if which == "k" else pool.v)[pages]                    # [P, nkv, page, hd]
    P, nkv, page, hd = data.shape
    if pool.kv_dtype == 0:
        vals = data.float()
    else:
        sb = (pool.ksb if which == "k" else pool.vsb)[pages].cpu().numpy().view(np.uint32)
        sc = torch.from_numpy(O.bits_to_f32((sb & 0xFFFF).astype(np.uint16)))
        bi = torch.from_numpy(O.bits_to_f32((sb >> 16).astype(np.uint16)))
        q = data.cpu().float().view(P, nkv, page, hd // 64, 64)
        vals = torch.from_numpy(O.bf16_round((q * sc[..., None] + bi[..., None]).view(P, nkv, page, hd).numpy()))
    return vals.cpu().permute(0, 2, 1, 3).reshape(P * page, nkv, hd)[:n]


def _random_case(dev, kv_dtype, lens, W, max_ctx, nq=8, nkv=2, hd=128, page=64):
    """A pool of random stored K/V (8-bit: random codes with scale ~ U(0.005, 0.02), bias ~
    U(-1.5, -0.5)) and random queries for rows of the given lengths."""
    B = len(lens)
    g = torch.Generator().manual_seed(sum(lens) + W + kv_dtype + 7 * nkv)
    pool = Pool(B, nkv, hd, max_ctx, page, kv_dtype, dev, seed=W + nkv)
    if kv_dtype == 0:
        pool.k.copy_(torch.randn(pool.k.shape, generator=g).to(torch.bfloat16))
        pool.v.copy_(torch.randn(pool.v.shape, generator=g).to(torch.bfloat16))
    else:
        pool.k.copy_(torch.randint(0, 256, pool.k.shape, generator=g, dtype=torch.uint8))
        pool.v.copy_(torch.randint(0, 256, pool.v.shape, generator=g, dtype=torch.uint8))

        def sbv():   # bf16 pairs packed scale | bias << 16
            sc = (0.005 + 0.015 * torch.rand(pool.ksb.shape, generator=g)).to(torch.bfloat16).view(torch.int16)
            bb = (-1.5 + torch.rand(pool.ksb.shape, generator=g)).to(torch.bfloat16).view(torch.int16)
            return (sc.to(torch.int32) & 0xFFFF) | (bb.to(torch.int32) << 16)
        pool.ksb.copy_(sbv())
        pool.vsb.copy_(sbv())
    q = torch.randn(B * W, nq * hd, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    return dict(pool=pool, q=q, qd=q.to(dev), sl=sl, B=B, W=W, nq=nq, nkv=nkv, hd=hd, page=page,
                max_ctx=max_ctx, kv_dtype=kv_dtype, lens=lens)


def _run_case(c, out=None, window=0):
    from mlx_dspark.ops import attention
    p = c["pool"]
    return attention(c["qd"], c["B"], c["W"], c["nq"], c["nkv"], c["hd"], c["hd"] ** -0.5, c["sl"], c["max_ctx"],
                     p.block_table, c["page"], c["kv_dtype"], p.k, p.v, p.ksb, p.vsb, causal=True, window=window,
                     out=out)


def _check_case(c, out, window=0):
    B, W, nq, nkv, hd = c["B"], c["W"], c["nq"], c["nkv"], c["hd"]
    G = nq // nkv
    scale = hd ** -0.5
    for b, L0 in enumerate(c["lens"]):
        K = _read_tokens(c["pool"], b, L0 + W, "k")
        V = _read_tokens(c["pool"], b, L0 + W, "v")
        qb = c["q"].view(B, W, nq, hd)[b].float()
        ref = torch.empty(W, nq, hd)
        j = torch.arange(L0 + W)[None, :]
        i = torch.arange(W)[:, None]
        hidden = j > L0 + i
        if window:
            hidden = hidden | (j <= L0 + i - window)      # query at L0 + i sees keys > L0 + i - window
        for h in range(nq):
            s = (qb[:, h] @ K[:, h // G].T) * scale
            s = s.masked_fill(hidden, float("-inf"))
            ref[:, h] = torch.softmax(s, -1) @ V[:, h // G]
        got = out.view(B, W, nq, hd)[b].float().cpu()
        err = (got - ref).abs().max().item()
        assert err < 2e-2, (b, err)


@pytest.mark.parametrize("kv_dtype", [0, 1])
@pytest.mark.parametrize("lens,W,max_ctx", [([4096], 16, 5184), ([3000, 5000], 9, 5200), ([100], 16, 8000),
                                            ([6000, 1000], 16, 12288), ([0, 64, 127], 4, 3500),
                                            ([0, 130], 16, 300), ([8100], 4, 8192), ([4096], 17, 4200),
                                            ([300, 2000], 20, 2100)])
def test_attention_streamed_splits(dev, kv_dtype, lens, W, max_ctx):
    """Long contexts: each split streams several key blocks (the split size grows with max_ctx),
    with ragged rows, splits past a row's length, a causal edge inside a block and rows whose
    keys end mid-block; against a float32 softmax over the stored K/V."""
    print(f"attn streamed kv={kv_dtype} lens={lens} W={W} max_ctx={max_ctx}", flush=True)
    c = _random_case(dev, kv_dtype, lens, W, max_ctx)
    out = _run_case(c)
    torch.cuda.synchronize()
    _check_case(c, out)


@pytest.mark.parametrize("kv_dtype", [0, 1])
def test_attention_interleaved_shapes_repeat(dev, kv_dtype):
    """Calls of different shapes (rows, kv heads, split counts) interleaved on the shared split
    workspace, each output cleared first, repeat bit for bit and match the float32 softmax."""
    print(f"attn interleaved kv={kv_dtype}", flush=True)
    cases = [_random_case(dev, kv_dtype, [4096], 16, 5184),
             _random_case(dev, kv_dtype, [700, 2500, 30], 9, 3000, nq=16, nkv=4),
             _random_case(dev, kv_dtype, [1500, 64], 16, 2048, nq=8, nkv=1)]
    first = []
    for rep in range(3):
        for k, c in enumerate(cases):
            out = torch.full((c["B"] * c["W"], c["nq"] * c["hd"]), float("nan"), dtype=torch.bfloat16, device=dev)
            _run_case(c, out=out)
            torch.cuda.synchronize()
            if rep == 0:
                _check_case(c, out)
                first.append(out.clone())
            else:
                assert torch.equal(out, first[k]), (rep, k)


@pytest.mark.parametrize("kv_dtype", [0, 1])
@pytest.mark.parametrize("lens,W,max_ctx,window", [([8192], 9, 8208, 0), ([8192], 9, 8208, 1024),
                                                   ([3000, 70], 16, 3100, 0), ([100, 1030], 9, 1200, 1024),
                                                   ([0, 64], 4, 200, 0), ([500], 1, 640, 64), ([300], 9, 400, 0),
                                                   ([5000], 17, 5100, 0), ([2000, 40], 32, 2100, 1024)])
def test_attention_head_dim_256(dev, kv_dtype, lens, W, max_ctx, window):
    """head_dim 256 verify passes (the Gemma-style shape: 16 query / 8 kv heads, 9 new tokens,
    an 8192-key global layer and 1024-key sliding windows), ragged rows, rows shorter than a
    window, single-token rows and a short context split into two query-tile groups; against a float32 softmax over the stored K/V with the
    window's mask (a query at position p sees keys p - window + 1 .. p)."""
    print(f"attn hd256 kv={kv_dtype} lens={lens} W={W} max_ctx={max_ctx} window={window}", flush=True)
    c = _random_case(dev, kv_dtype, lens, W, max_ctx, nq=16, nkv=8, hd=256)
    out = _run_case(c, window=window)
    torch.cuda.synchronize()
    _check_case(c, out, window=window)


@pytest.mark.parametrize("kv_dtype", [0, 1])
@pytest.mark.parametrize("lens,W,max_ctx,window", [([3000, 200, 5000], 16, 5200, 1024), ([4100], 9, 4200, 300),
                                                   ([700, 700], 4, 1024, 256)])
def test_attention_sliding_window_head_dim_128(dev, kv_dtype, lens, W, max_ctx, window):
    """head_dim 128 verify passes with a sliding window: only the splits of one window are
    launched, each row's starting where its first row's window starts (ragged rows start at
    different splits, windows that begin on and off a split boundary)."""
    print(f"attn window hd128 kv={kv_dtype} lens={lens} W={W} max_ctx={max_ctx} window={window}", flush=True)
    c = _random_case(dev, kv_dtype, lens, W, max_ctx)
    out = _run_case(c, window=window)
    torch.cuda.synchronize()
    _check_case(c, out, window=window)


@pytest.mark.parametrize("kv_dtype", [0, 1])
@pytest.mark.parametrize("lens,W,max_ctx", [([4096], 16, 4200), ([8192, 3000], 16, 8300),
                                            ([5000, 100, 2000, 7000], 9, 7100), ([4096], 17, 4200)])
def test_attention_qwen3_8b_heads(dev, kv_dtype, lens, W, max_ctx):
    """The Qwen3-8B head shape (32 query / 8 kv heads): four 16-row query tiles per kv head in
    two passes of two (3- and 5-tile row groups included), ragged rows over long contexts."""
    print(f"attn 32/8 heads kv={kv_dtype} lens={lens} W={W} max_ctx={max_ctx}", flush=True)
    c = _random_case(dev, kv_dtype, lens, W, max_ctx, nq=32, nkv=8)
    out = _run_case(c)
    torch.cuda.synchronize()
    _check_case(c, out)


@pytest.mark.parametrize("kv_dtype", [0, 1])
@pytest.mark.parametrize("lens,W,max_ctx,window", [([768], 9, 841, 0), ([700, 40], 9, 800, 0), ([760], 9, 841, 256),
                                                   ([500, 0], 1, 640, 0), ([1000], 9, 2100, 0)])
def test_attention_qwen3_06b_heads(dev, kv_dtype, lens, W, max_ctx, window):
    """The Qwen3-0.6B head shape (16 query / 8 kv heads, 9 new tokens: two query tiles per kv
    head). Grids of at most 64 (row, kv head, 256-key split) workgroups run 128-key splits (the
    first four cases, ragged rows, a sliding window and single-token rows included); the last
    case's 72 run 256-key splits."""
    print(f"attn 16/8 heads kv={kv_dtype} lens={lens} W={W} max_ctx={max_ctx} window={window}", flush=True)
    c = _random_case(dev, kv_dtype, lens, W, max_ctx, nq=16, nkv=8)
    out = _run_case(c, window=window)
    torch.cuda.synchronize()
    _check_case(c, out, window=window)
