"""GPU parity of the Gemma-style target layout (embedding scale, sandwich norms, GeGLU,
5:1 sliding-window / global layers with their own RoPE bases, final soft-cap 30): the
verify forward against the oracle past the window, greedy speculative decoding reproducing
the oracle's greedy stream, seeded sampled decoding at the G12 decoding settings, and a
batched SpecSlots round."""

import numpy as np
import pytest
import torch

from _parity import Twin, check_logits, check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2   # greedy-stream margin rule (normalised logits)


@pytest.fixture(scope="module")
def gemma(dev):
    from mlx_dspark import synthetic
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    model = synthetic.build_target("tiny-gemma", seed=8, keep_mlx=True)
    d, cfg = synthetic.build_dspark(model.args, seed=9, keep_mlx=True, num_hidden_layers=1, block_size=8,
                                    taps=[1, 3, 5])
    tok = SyntheticTokenizer(model.args.vocab_size)
    return Target(model, tok), tok, d, cfg


@pytest.mark.parametrize("kv_bits", [None, 8])
def test_gemma_forward_past_the_window(dev, gemma, kv_bits):
    target, tok, d, cfg = gemma
    model = target.model
    a = model.args
    assert a.sandwich_norms and a.window(0) == 32 and a.window(5) == 0 and a.final_logit_softcapping == 30.0
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, a.vocab_size, 90).tolist()       # longer than the 32-token window
    cache = model.make_cache(max_ctx=256, kv_bits=kv_bits)
    logits, fused = model.prefill(prompt, cache, [1, 5])
    ref = Twin(lambda: OM.OracleTarget(model, kv_bits=kv_bits))
    (rl, rf), (el, _) = ref.forward(prompt, [1, 5])
    check_logits(logits[0, -1], rl[-1], "prefill last row", exact=el[-1])
    assert (fused[0].float().cpu() - rf).abs().max() < 0.05 * rf.abs().max()
    assert float(logits.abs().max()) <= 30.0
    block = rng.integers(0, a.vocab_size, 9).tolist()
    vl, _ = model.forward(torch.tensor([block], dtype=torch.int32, device=dev), cache, None, advance=False)
    (rvl, _), (evl, _) = ref.forward(block)
    check_logits(vl[0], rvl, "verify block", exact=evl)


def test_gemma_window_masks_old_keys(dev, gemma):
    """A sliding layer must not see keys older than the window: an oracle without windows
    disagrees with the engine, the windowed oracle agrees."""
    target, tok, d, cfg = gemma
    model = target.model
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, model.args.vocab_size, 120).tolist()
    cache = model.make_cache(max_ctx=256)
    lg, _ = model.prefill(prompt, cache)
    (good, _), (good_ex, _) = Twin(lambda: OM.OracleTarget(model)).forward(prompt)
    good, good_ex = good[-1], good_ex[-1]
    bad_t = OM.OracleTarget(model)
    bad_t.a = type(model.args)(**{**model.args.__dict__, "sliding_window": None})
    bad = bad_t.forward(prompt)[0][-1]
    nrm = lambda x: x / x.pow(2).mean().sqrt()
    d_good = float((nrm(lg[0, -1].float().cpu()) - nrm(good)).abs().max())
    d_bad = float((nrm(lg[0, -1].float().cpu()) - nrm(bad)).abs().max())
    print(f"windowed oracle {d_good:.4f}, unwindowed oracle {d_bad:.4f}", flush=True)
    bound = check_logits(lg[0, -1], good, "windowed oracle", exact=good_ex)
    assert d_bad > 2 * bound


def test_gemma_speculative_greedy_stream(dev, gemma):
    from mlx_dspark.generate import speculative_generate
    target, tok, d, cfg = gemma
    target.verify_tap()
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, target.model.args.vocab_size, 50).tolist()
    res = speculative_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=24, max_draft_tokens=8,
                               lookup_drafts=False)
    check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    assert sum(res.accept_lengths) + 1 == res.num_tokens


def test_gemma_sampled_g12_settings_seeded(dev, gemma):
    """The G12 decoding settings: k = 8, temperature 1.0, top-p 0.95, seeded."""
    from mlx_dspark.generate import speculative_generate
    target, tok, d, cfg = gemma
    kw = dict(prompt_ids=list(range(40)), max_new_tokens=20, temperature=1.0, top_p=0.95, max_draft_tokens=8,
              lookup_drafts=False)
    a = speculative_generate(target, tok, d, seed=7, **kw)
    b = speculative_generate(target, tok, d, seed=7, **kw)
    assert a.token_ids == b.token_ids and sum(a.accept_lengths) + 1 == a.num_tokens


def test_gemma_batched_slots(dev, gemma):
    from mlx_dspark.batch_engine import batch_spec_generate, batchable
    target, tok, d, cfg = gemma
    assert batchable(target)
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, target.model.args.vocab_size, n).tolist() for n in (40, 70)]
    res = batch_spec_generate(target, tok, d, prompts, max_new_tokens=12, max_draft_tokens=4)
    for p, r in zip(prompts, res):
        check_greedy_stream(target.model, p, r.token_ids, MIN_MATCH)
