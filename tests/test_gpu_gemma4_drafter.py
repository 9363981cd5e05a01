"""GPU parity of the gemma4-family DSpark drafter (src/mlx_dspark/model.py, config.py): head_dim
512 attention over one global kv head, V = v_norm(k_proj) with k_eq_v, proportional RoPE,
sandwich norms with layer_scalar, tanh-GeLU, soft-cap 30 and the sqrt(hidden) embedding scale;
against the oracle, and greedy speculative decoding on the Gemma-style target reproducing the
oracle's greedy stream."""

import numpy as np
import pytest
import torch

from _parity import Twin, check_logits, check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2


def _ref_attention(q, K, V, scale, L0, causal):
    """q [W, nq, hd], K/V [L0 + W, nkv, hd] float32 -> [W, nq, hd]"""
    W, nq, hd = q.shape
    G = nq // K.shape[1]
    out = torch.empty(W, nq, hd)
    j = torch.arange(L0 + W)[None, :]
    i = torch.arange(W)[:, None]
    for h in range(nq):
        s = (q[:, h] @ K[:, h // G].T) * scale
        if causal:
            s = s.masked_fill(j > L0 + i, float("-inf"))
        out[:, h] = torch.softmax(s, -1) @ V[:, h // G]
    return out


@pytest.mark.parametrize("lens,W,nq,causal", [([0], 7, 16, False), ([40, 300], 7, 16, False), ([130], 9, 4, True),
                                              ([2000], 16, 16, False)])
def test_attention_head_dim_512(dev, lens, W, nq, causal):
    """head_dim 512 (bf16 KV, one kv head): query-tile groups on the grid, split partials
    combined, against a float32 softmax over the stored K/V."""
    from mlx_dspark.ops import attention
    print(f"attn hd512 lens={lens} W={W} nq={nq} causal={causal}", flush=True)
    B, nkv, hd, page = len(lens), 1, 512, 64
    max_ctx = max(lens) + W + 64
    mp = (max_ctx + page - 1) // page
    g = torch.Generator().manual_seed(sum(lens) + W + nq)
    n_pages = B * mp + 2
    bt = torch.randperm(n_pages, generator=g)[: B * mp].view(B, mp).to(torch.int32)
    kp = torch.randn(n_pages, nkv, page, hd, generator=g).to(torch.bfloat16)
    vp = torch.randn(n_pages, nkv, page, hd, generator=g).to(torch.bfloat16)
    q = (torch.randn(B * W, nq * hd, generator=g) * hd ** -0.25).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    out = attention(q.to(dev), B, W, nq, nkv, hd, 1.0 / 16, sl.to(dev), max_ctx, bt.to(dev), page, 0, kp.to(dev),
                    vp.to(dev), causal=causal)
    torch.cuda.synchronize()
    for b, L0 in enumerate(lens):
        n = L0 + W
        idx = torch.arange(n)
        pages = bt[b][idx // page].long()
        K = kp[pages, :, idx % page].float()
        V = vp[pages, :, idx % page].float()
        ref = _ref_attention(q.view(B, W, nq, hd)[b].float(), K, V, 1.0 / 16, L0, causal)
        got = out.view(B, W, nq, hd)[b].float().cpu()
        err = (got - ref).abs().max().item()
        assert err < 2e-2, (b, err)


def test_append_v_norm_and_proportional_rope(dev):
    """dsk_qkv_norm_rope_append at head_dim 512: K = rope(k_norm(k)) with the proportional table,
    V = RMSNorm(v) (unit weight), queries normed and roped, against float32 closed forms."""
    from mlx_dspark import ops
    B, W, nq, nkv, hd, page = 1, 7, 4, 1, 512, 16
    L0 = 5
    max_ctx = 64
    mp = max_ctx // page
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(B * W, (nq + 2 * nkv) * hd, generator=g).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(hd, generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(hd, generator=g)).to(torch.bfloat16)
    vn = torch.ones(hd, dtype=torch.bfloat16)
    inv = ops.rope_inv_freq(hd, 1e6, dev, rotary_fraction=0.25)
    bt = torch.arange(mp, dtype=torch.int32).view(1, mp).to(dev)
    kp = torch.zeros(mp, nkv, page, hd, dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    sl = torch.tensor([L0], dtype=torch.int32, device=dev)
    qo = ops.qkv_rope_append(qkv.to(dev), B, W, nq, nkv, hd, qn.to(dev), kn.to(dev), 1e-6, inv, sl, bt, page, 0, kp,
                             vp, v_norm=vn.to(dev))
    torch.cuda.synchronize()
    x = qkv.float().view(W, nq + 2 * nkv, hd)
    pos = torch.arange(L0, L0 + W)
    invc = OM.inv_freq(hd, 1e6, 0.25)
    q_ref = OM.bf(OM.rope(OM.bf(OM.rmsnorm(x[:, :nq], qn.float(), 1e-6)).transpose(0, 1), pos, 0, invc).transpose(0, 1))
    k_ref = OM.bf(OM.rope(OM.bf(OM.rmsnorm(x[:, nq:nq + 1], kn.float(), 1e-6)).transpose(0, 1), pos, 0, invc)
                  .transpose(0, 1))
    v_ref = OM.bf(OM.rmsnorm(x[:, nq + 1:], torch.ones(hd), 1e-6))
    tok = torch.arange(L0, L0 + W)
    k_got = kp[tok // page, :, tok % page].float().cpu()
    v_got = vp[tok // page, :, tok % page].float().cpu()
    tol = lambda r: 2 ** -7 * r.abs().max()
    assert (qo.float().cpu().view(W, nq, hd) - q_ref).abs().max() <= tol(q_ref)
    assert (k_got - k_ref).abs().max() <= tol(k_ref)
    assert (v_got - v_ref).abs().max() <= tol(v_ref)
    # the un-rotated dims (frequency 0) of K are the normed projection itself
    kn_only = OM.bf(OM.rmsnorm(x[:, nq:nq + 1], kn.float(), 1e-6))
    assert torch.equal(k_ref[..., 64:256], kn_only[..., 64:256])


@pytest.fixture(scope="module")
def gemma4_pair(dev):
    from mlx_dspark import synthetic
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    model = synthetic.build_target("tiny-gemma", seed=8, keep_mlx=True)
    d, cfg = synthetic.build_dspark(model.args, seed=13, keep_mlx=True, num_hidden_layers=2, block_size=7,
                                    taps=[1, 3, 5], family="gemma4")
    tok = SyntheticTokenizer(model.args.vocab_size)
    return Target(model, tok), tok, d, cfg


def test_gemma4_drafter_matches_oracle(dev, gemma4_pair):
    target, tok, d, cfg = gemma4_pair
    assert cfg.family == "gemma4" and cfg.attn_head_dim == 512 and cfg.n_kv_heads == 1 and cfg.scaling == 1.0
    model = target.model
    rng = np.random.default_rng(4)
    V = model.args.vocab_size
    prompt = rng.integers(0, V, 45).tolist()
    cache = model.make_cache(max_ctx=256)
    _, fused = model.prefill(prompt, cache, list(cfg.target_layer_ids))
    dcache = d.make_ctx_cache(max_ctx=256)
    d.update_context(fused[0], 0, dcache)
    oa = Twin(lambda: OM.OracleDSpark(d))
    oa.update_context(fused[0].float().cpu())
    # context K/V in the drafter cache against the oracle's
    k_pool, v_pool, _, _ = dcache.layer_args(0)
    bt = dcache.block_table[0].cpu()
    idx = torch.arange(45)
    pages = bt[idx // dcache.page].long()
    kg = k_pool[pages.to(dev), :, (idx % dcache.page).to(dev)].float().cpu()
    vg = v_pool[pages.to(dev), :, (idx % dcache.page).to(dev)].float().cpu()
    assert (kg - oa.f32.K[0]).abs().max() <= 0.02 * oa.f32.K[0].abs().max()
    assert (vg - oa.f32.V[0]).abs().max() <= 0.02 * oa.f32.V[0].abs().max()
    block = torch.tensor([[int(prompt[-1])] + [cfg.mask_token_id] * (cfg.block_size - 1)], dtype=torch.int32,
                         device=dev)
    got = d.block_logits(block, dcache, 5)[0]
    want, ex = oa.base_logits(block.cpu()[0], 5)
    check_logits(got, want, "gemma4 drafter block logits", exact=ex)
    assert float(got.abs().max()) <= 30.0


@pytest.mark.parametrize("graph", [True, False])
def test_speculative_generate_gemma4_drafter(dev, gemma4_pair, graph):
    from mlx_dspark.generate import speculative_generate
    target, tok, d, cfg = gemma4_pair
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, target.model.args.vocab_size, 30).tolist()
    print(f"spec gemma4 drafter graph={graph}", flush=True)
    res = speculative_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=16, max_draft_tokens=4,
                               lookup_drafts=False, use_graph=graph)
    check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    assert res.num_tokens >= 16 and sum(res.accept_lengths) + 1 == res.num_tokens
