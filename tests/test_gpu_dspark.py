"""GPU parity of the DSpark path: the Markov block-sampling kernel (greedy and sampled) and
the drafter forward against the oracle, and speculative_generate reproducing the oracle's
greedy stream (fast graph path, two-phase paths with penalties and confidence truncation,
lookup rounds), seeded sampling."""

import numpy as np
import pytest
import torch

from oracle import accept as OA
from _parity import Twin, check_logits, check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2   # greedy-stream margin rule (normalised logits)


def _w8(N, K, seed, dev, keep=True):
    from mlx_dspark.ops import W8Weight
    g = torch.Generator().manual_seed(seed)
    q, s, b = W8Weight.quantize_mlx((torch.randn(N, K, generator=g) * 0.05).to(dev))
    W = W8Weight.from_mlx(q, s, b)
    W.mlx = (q, s, b)
    return W


def _table(V, R, seed, dev):
    from mlx_dspark.ops import W8Table, W8Weight
    g = torch.Generator().manual_seed(seed)
    q, s, b = W8Weight.quantize_mlx((torch.randn(V, R, generator=g) * 0.3).to(dev))
    return W8Table(q, s, b)


@pytest.mark.parametrize("B,cap,V", [(1, 8, 4096), (3, 5, 151936 // 4), (1, 2, 1024), (20, 3, 4096)])
def test_markov_greedy_matches_oracle(dev, B, cap, V):
    from mlx_dspark import ops
    print(f"markov greedy B={B} cap={cap} V={V}", flush=True)
    w1 = _table(V, 256, 11, dev)
    w2 = _w8(V, 256, 12, dev)
    g = torch.Generator().manual_seed(B * cap)
    base = torch.randn(B, cap, V, generator=g) * 2.0
    first = torch.randint(0, V, (B,), generator=g).to(torch.int32)
    tok = ops.markov_block(base.to(dev), first.to(dev), w1, w2).cpu()
    o = OM.OracleDSpark.__new__(OM.OracleDSpark)
    o.w1, o.w2 = OM.deq_table(w1), OM.deq(w2)
    for b in range(B):
        prev = int(first[b])
        for i in range(cap):
            row = o.step_logits(base[b, i], prev)            # oracle logits given the engine's prev
            t = int(tok[b, i])
            top = float(row.max())
            # the engine's token is the oracle argmax, or within one bf16 ulp of the max
            assert t == int(torch.argmax(row)) or float(row[t]) >= top - abs(top) * 2 ** -7, (b, i)
            prev = t


@pytest.mark.parametrize("B", [2, 20])
def test_markov_sampled_matches_oracle_sampling(dev, B):
    """B = 20 runs as pieces of 16 rows: every row still draws from its own Philox row."""
    from mlx_dspark import ops
    cap, V = 4, 8192
    print(f"markov sampled B={B}", flush=True)
    w1 = _table(V, 256, 21, dev)
    w2 = _w8(V, 256, 22, dev)
    g = torch.Generator().manual_seed(5)
    base = torch.randn(B, cap, V, generator=g)
    first = torch.tensor([3, 4000] + [(977 * b) % V for b in range(2, B)], dtype=torch.int32)
    tok, ql = ops.markov_block(base.to(dev), first.to(dev), w1, w2, temperature=0.8, top_p=0.9, top_k=0, seed=77,
                               offset=3)
    tok, ql = tok.cpu(), ql.cpu()
    o = OM.OracleDSpark.__new__(OM.OracleDSpark)
    o.w1, o.w2 = OM.deq_table(w1), OM.deq(w2)
    for b in range(B):
        prev = int(first[b])
        for i in range(cap):
            row = o.step_logits(base[b, i], prev)
            assert (ql[b, i] - row).abs().max() <= row.abs().max() * 2 ** -7   # same logits up to an ulp
            # given the engine's logits, the draw is bit-exact with the oracle's sampler
            t_ref, _ = OA.sample_rows(ql[b, i].numpy()[None], 0.8, 0.9, 0, mul_inv=True, seed=77, offset=3,
                                      row0=b * cap + i)
            assert int(tok[b, i]) == int(t_ref[0])
            prev = int(tok[b, i])


@pytest.fixture(scope="module")
def pair(dev):
    from mlx_dspark import synthetic
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    model = synthetic.build_target("tiny", seed=3, keep_mlx=True)
    d, cfg = synthetic.build_dspark(model.args, seed=4, keep_mlx=True, num_hidden_layers=1, block_size=7,
                                    taps=[0, 2, 3])
    tok = SyntheticTokenizer(model.args.vocab_size)
    return Target(model, tok), tok, d, cfg


def test_dspark_drafter_matches_oracle(dev, pair):
    target, tok, d, cfg = pair
    model = target.model
    rng = np.random.default_rng(1)
    V = model.args.vocab_size
    prompt = rng.integers(0, V, 45).tolist()
    cache = model.make_cache(max_ctx=256)
    _, fused = model.prefill(prompt, cache, list(cfg.target_layer_ids))
    dcache = d.make_ctx_cache(max_ctx=256)
    d.update_context(fused[0], 0, dcache)
    oa = Twin(lambda: OM.OracleDSpark(d))
    oa.update_context(fused[0].float().cpu())
    od = oa.f32
    block = torch.tensor([[int(prompt[-1])] + [cfg.mask_token_id] * (cfg.block_size - 1)], dtype=torch.int32,
                         device=dev)
    got = d.block_logits(block, dcache, 4)[0]
    want, ex = oa.base_logits(block.cpu()[0], 4)
    check_logits(got, want, "dspark block logits", exact=ex)
    # the reference-shaped entry points agree with the fused one
    noise = d.embed(block)
    hid = d.backbone(noise, dcache.lengths[0], dcache)
    lg = d.compute_logits(hid[:, :4])[0]
    assert OM.normalized_maxdiff(lg, got) < 1e-2
    # the confidence head on the normed rows
    conf = d.confidence_logits(hid[0, :4], [int(prompt[-1]), 5, 6, 7])
    cref = od.confidence_logits(od.block_hidden(block.cpu()[0])[:4], [int(prompt[-1]), 5, 6, 7])
    assert (conf.cpu() - cref).abs().max() < 0.05 * (cref.abs().max() + 1e-3) + 1e-2


@pytest.mark.parametrize("cap,lookup,graph,conf", [(2, False, True, 0.0), (None, False, True, 0.0),
                                                   (3, True, False, 0.0), (4, False, False, 0.3)])
def test_speculative_generate_reproduces_greedy_stream(dev, pair, cap, lookup, graph, conf):
    from mlx_dspark.generate import speculative_generate
    target, tok, d, cfg = pair
    rng = np.random.default_rng(2)
    base = rng.integers(0, target.model.args.vocab_size, 12).tolist()
    prompt = base + base + base[:6]            # repeats so lookup rounds fire
    print(f"spec cap={cap} lookup={lookup} graph={graph} conf={conf}", flush=True)
    res = speculative_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=20, max_draft_tokens=cap,
                               lookup_drafts=lookup, use_graph=graph, confidence_threshold=conf)
    check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    assert res.num_tokens >= 20 and sum(res.accept_lengths) + 1 == res.num_tokens
    assert res.target_forwards == res.num_rounds + 1
    if lookup:
        assert res.lookup_rounds > 0


def test_speculative_generate_penalties_match_penalised_greedy(dev, pair):
    from mlx_dspark.generate import speculative_generate
    target, tok, d, cfg = pair
    prompt = list(range(30, 50))
    res = speculative_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=16, max_draft_tokens=3,
                               lookup_drafts=False, presence_penalty=0.8, frequency_penalty=0.5)
    ot = OM.OracleTarget(target.model)
    logits, _ = ot.forward(prompt)
    counts: dict = {}
    out = []
    row = logits[-1]
    for i in range(len(res.token_ids)):
        pen = torch.zeros_like(row)
        for t, v in OM.penalty_rows(counts, 0.8, 0.5, [])[0].items():
            pen[t] = v
        r = row - pen
        rn = r / r.pow(2).mean().sqrt()
        top2 = torch.topk(rn, 2).values
        t = int(torch.argmax(r))
        if t != res.token_ids[i]:
            assert float(top2[0] - top2[1]) <= TOL, i
            assert i >= MIN_MATCH, f"only {i} tokens match the penalised oracle"
            break
        out.append(t)
        counts[t] = counts.get(t, 0) + 1
        row = ot.forward([t])[0][-1]


def test_speculative_generate_sampled_is_seeded(dev, pair):
    from mlx_dspark.generate import speculative_generate
    target, tok, d, cfg = pair
    kw = dict(prompt_ids=list(range(20)), max_new_tokens=16, temperature=0.8, top_p=0.9, seed=123,
              lookup_drafts=False, max_draft_tokens=4)
    a = speculative_generate(target, tok, d, **kw)
    b = speculative_generate(target, tok, d, **kw)
    c = speculative_generate(target, tok, d, **{**kw, "seed": 124})
    assert a.token_ids == b.token_ids
    assert a.token_ids != c.token_ids
    assert sum(a.accept_lengths) + 1 == a.num_tokens
