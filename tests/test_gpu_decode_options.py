"""GPU parity of the decode options around the verify path: per-token logprobs (the
row log-softmax / top-k kernel against a float64 CPU log-softmax with a stable
value-then-index order), greedy_generate with penalties and logprobs against the oracle,
speculative_generate logprobs (graph round, lookup round, penalised round) against the
one-token loop, and prompt-lookup decoding (lookup_generate) reproducing the oracle's greedy
stream, reusing a cached prefix and sampling reproducibly from its seed."""

import numpy as np
import pytest
import torch

from _parity import check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2          # greedy-stream margin rule (normalised logits)
LP_TOL = 5e-2       # logprob agreement between two engine paths (different verify widths)


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


def _cpu_logprobs(x: np.ndarray, tokens, k):
    x64 = x.astype(np.float64)
    m = x64.max(-1, keepdims=True)
    lp = x64 - m - np.log(np.exp(x64 - m).sum(-1, keepdims=True))
    chosen = lp[np.arange(len(tokens)), tokens]
    ids = np.stack([np.lexsort((np.arange(x.shape[1]), -x[r]))[:k] for r in range(x.shape[0])])
    return chosen, ids, np.take_along_axis(lp, ids, -1)


@pytest.mark.parametrize("R,V,k", [(5, 151936, 20), (3, 1000, 64), (2, 70, 0), (4, 262144, 5)])
def test_row_logprobs_matches_log_softmax(dev, R, V, k):
    from mlx_dspark import ops
    rng = np.random.default_rng(R * 7 + V)
    x = (rng.standard_normal((R, V)) * 4).astype(np.float32)
    x[0, 10:14] = x[0].max() + 1.0            # a four-way tie at the top: ordered by token id
    x[1, ::3] = -np.inf                        # masked entries
    tokens = rng.integers(0, V, R)
    tokens[1] = 1                              # a finite entry of the masked row
    print(f"row_logprobs R={R} V={V} k={k}", flush=True)
    chosen, ids, vals = ops.row_logprobs(torch.from_numpy(x).to(dev), torch.from_numpy(tokens).to(dev), k)
    c_ref, i_ref, v_ref = _cpu_logprobs(x, tokens, k)
    np.testing.assert_allclose(chosen.cpu().numpy(), c_ref, rtol=0, atol=2e-4)
    if k:
        assert (ids.cpu().numpy() == i_ref).all()
        np.testing.assert_allclose(vals.cpu().numpy(), v_ref, rtol=0, atol=2e-4)
        assert ids.cpu()[0, :4].tolist() == [10, 11, 12, 13]
    # strided rows (a view into a wider buffer) read the same values
    wide = torch.zeros((R, V + 64), device=dev)
    wide[:, :V] = torch.from_numpy(x).to(dev)
    c2, _, _ = ops.row_logprobs(wide[:, :V], torch.from_numpy(tokens).to(dev), 0)
    assert torch.equal(c2, chosen)


def _oracle_penalised_greedy(model, prompt, n, presence, frequency):
    """Oracle greedy decoding with OpenAI penalties over the tokens emitted so far; returns
    tokens, margins and the raw log-softmax rows at every decision."""
    ot = OM.OracleTarget(model)
    row = ot.forward(prompt)[0][-1]
    counts: dict = {}
    toks, margins, lps = [], [], []   # lps: (raw log-softmax row, raw row RMS)
    for _ in range(n):
        pen = torch.zeros_like(row)
        for t, v in OM.penalty_rows(counts, presence, frequency, [])[0].items():
            pen[t] = v
        r = row - pen
        rn = r / r.pow(2).mean().sqrt()
        top2 = torch.topk(rn, 2).values
        margins.append(float(top2[0] - top2[1]))
        lps.append((torch.log_softmax(row.double(), -1), float(row.pow(2).mean().sqrt())))
        t = int(torch.argmax(r))
        toks.append(t)
        counts[t] = counts.get(t, 0) + 1
        row = ot.forward([t])[0][-1]
    return toks, margins, lps


@pytest.mark.parametrize("presence,frequency", [(0.0, 0.0), (0.8, 0.5)])
def test_greedy_generate_penalties_and_logprobs(dev, pair, presence, frequency):
    from mlx_dspark.generate import greedy_generate
    target, tok, d, cfg = pair
    prompt = list(range(30, 50))
    print(f"greedy_generate presence={presence} frequency={frequency}", flush=True)
    res = greedy_generate(target, tok, prompt_ids=prompt, max_new_tokens=14, presence_penalty=presence,
                          frequency_penalty=frequency, logprobs=4)
    assert res.num_tokens == 14 and len(res.logprobs) == 14
    ref, margins, lps = _oracle_penalised_greedy(target.model, prompt, 14, presence, frequency)
    for i, (a, b) in enumerate(zip(res.token_ids, ref)):
        e = res.logprobs[i]
        assert e["token_id"] == a and len(e["top"]) == 4
        vals = [v for _, v in e["top"]]
        assert vals == sorted(vals, reverse=True) and sum(np.exp(vals)) <= 1.0 + 1e-5
        # raw (unpenalised) target distribution; the logits agree to TOL of the row RMS, so a
        # logprob (a logit minus the log-sum-exp) agrees to twice that
        lp_ref, rms = lps[i]
        assert abs(e["logprob"] - float(lp_ref[a])) < 2 * TOL * rms + 1e-3, (i, e["logprob"], float(lp_ref[a]))
        if presence == 0.0 and frequency == 0.0:
            assert e["top"][0][0] == a or abs(e["top"][0][1] - e["logprob"]) < 1e-6
        if a != b:
            assert margins[i] <= TOL, (i, a, b, margins[i])
            assert i >= MIN_MATCH, f"only {i} tokens match the penalised oracle"
            break


@pytest.mark.parametrize("lookup,graph,penalised", [(False, True, False), (True, False, False), (False, False, True)])
def test_speculative_generate_logprobs_match_one_token_loop(dev, pair, lookup, graph, penalised):
    from mlx_dspark.generate import greedy_generate, speculative_generate
    target, tok, d, cfg = pair
    rng = np.random.default_rng(2)
    base = rng.integers(0, target.model.args.vocab_size, 12).tolist()
    prompt = base + base + base[:6]
    pen = dict(presence_penalty=0.6, frequency_penalty=0.3) if penalised else {}
    print(f"spec logprobs lookup={lookup} graph={graph} penalised={penalised}", flush=True)
    res = speculative_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=18, max_draft_tokens=3,
                               lookup_drafts=lookup, use_graph=graph, logprobs=3, **pen)
    one = greedy_generate(target, tok, prompt_ids=prompt, max_new_tokens=len(res.token_ids), logprobs=3, **pen)
    assert len(res.logprobs) == res.num_tokens
    for i, (a, b) in enumerate(zip(res.token_ids, one.token_ids)):
        if a != b:
            break
        ea, eb = res.logprobs[i], one.logprobs[i]
        assert ea["token_id"] == a and abs(ea["logprob"] - eb["logprob"]) < LP_TOL, (i, ea, eb)
        assert [t for t, _ in ea["top"]][:1] == [t for t, _ in eb["top"]][:1] or \
            abs(ea["top"][0][1] - ea["top"][1][1]) < LP_TOL
    else:
        i = len(res.token_ids)
    assert i >= 8, "the two decoders diverged early"


def test_lookup_generate_reproduces_greedy_stream(dev, pair):
    from mlx_dspark.lookup import lookup_generate
    target, tok, d, cfg = pair
    rng = np.random.default_rng(5)
    base = rng.integers(0, target.model.args.vocab_size, 10).tolist()
    prompt = base * 3 + base[:5]
    res = lookup_generate(target, tok, prompt_ids=prompt, max_new_tokens=24, max_draft_tokens=5)
    check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    assert res.num_tokens >= 24 and sum(res.accept_lengths) + 1 == res.num_tokens
    assert res.lookup_rounds > 0 and res.target_forwards == res.num_rounds + 1


def test_lookup_generate_reuses_a_cached_prefix(dev, pair):
    from mlx_dspark.lookup import lookup_generate
    target, tok, d, cfg = pair
    rng = np.random.default_rng(6)
    prefix = rng.integers(0, target.model.args.vocab_size, 40).tolist()
    prompt = prefix + prefix[:8]
    cache = target.make_cache(max_ctx=256)
    target.model.prefill(prefix, cache)
    res = lookup_generate(target, tok, prompt_ids=prompt, cache=cache, reuse_len=len(prefix), max_new_tokens=12)
    check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    with pytest.raises(ValueError):
        lookup_generate(target, tok, prompt_ids=prompt, cache=target.make_cache(max_ctx=256), reuse_len=5)


def test_lookup_generate_sampled_is_seeded(dev, pair):
    from mlx_dspark.lookup import lookup_generate
    target, tok, d, cfg = pair
    base = list(range(100, 112))
    kw = dict(prompt_ids=base * 3, max_new_tokens=16, temperature=0.9, top_p=0.95)
    a = lookup_generate(target, tok, seed=11, **kw)
    b = lookup_generate(target, tok, seed=11, **kw)
    c = lookup_generate(target, tok, seed=12, **kw)
    assert a.token_ids == b.token_ids and a.token_ids != c.token_ids
    assert sum(a.accept_lengths) + 1 == a.num_tokens
