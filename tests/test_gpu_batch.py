"""GPU parity of continuous batching (SpecSlots, batch_spec_generate, batch_generate_baseline):
every row reproduces the oracle's greedy decoding of its own prompt (greedy-stream margin
rule), slot turnover (admit / retire with block-table compaction) keeps rows independent,
a shared prefix on shared pages gives token-identical results to private prefills, and the
sampled rounds are reproducible from the seed."""

import numpy as np
import pytest

from _parity import check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2   # greedy-stream margin rule (normalised logits)


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


def _check_greedy(model, prompt, tokens):
    check_greedy_stream(model, prompt, tokens, MIN_MATCH)


def _prompts(V, lens, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, V, n).tolist() for n in lens]


@pytest.mark.parametrize("batched_drafter", [True, False])
def test_batch_spec_generate_rows_follow_greedy(dev, pair, batched_drafter):
    from mlx_dspark.batch_engine import batch_spec_generate
    target, tok, d, cfg = pair
    prompts = _prompts(target.model.args.vocab_size, [20, 45, 33], 7)
    print(f"batch_spec_generate batched_drafter={batched_drafter}", flush=True)
    res = batch_spec_generate(target, tok, d, prompts, max_new_tokens=[16, 12, 20], max_draft_tokens=3,
                              batched_drafter=batched_drafter)
    for p, r, n in zip(prompts, res, [16, 12, 20]):
        assert r.num_tokens >= n and sum(r.accept_lengths) + 1 == r.num_tokens
        _check_greedy(target.model, p, r.token_ids)


def test_batch_wider_than_one_kernel_pass(dev, pair):
    """20 rows at once: the verify forward (20 x 4 rows), the drafter's block (20 x 7 rows) and
    context appends run as groups of whole rows of at most 64 rows, the Markov head in pieces of
    16 rows; every row still follows its own prompt's greedy decoding."""
    from mlx_dspark.batch_engine import batch_spec_generate
    target, tok, d, cfg = pair
    n = 20
    prompts = _prompts(target.model.args.vocab_size, [9 + 3 * i for i in range(n)], 13)
    print(f"batch_spec_generate over {n} rows", flush=True)
    res = batch_spec_generate(target, tok, d, prompts, max_new_tokens=[8] * n, max_draft_tokens=3)
    for p, r in zip(prompts, res):
        assert r.num_tokens >= 8 and sum(r.accept_lengths) + 1 == r.num_tokens
        _check_greedy(target.model, p, r.token_ids)


def test_spec_slots_turnover(dev, pair):
    """Capacity 2, five requests admitted as slots free up: rows retire at different rounds,
    compaction moves block-table rows, and every result still follows its own prompt."""
    from mlx_dspark.batch_engine import SpecSlots
    target, tok, d, cfg = pair
    prompts = _prompts(target.model.args.vocab_size, [17, 40, 9, 28, 50], 11)
    mnt = [6, 18, 10, 4, 14]
    slots = SpecSlots(target, tok, d, capacity=2, max_draft_tokens=2, max_ctx=256)
    pending = list(range(len(prompts)))
    results = {}
    rounds = 0
    while pending or slots.n_active:
        while pending and slots.has_free_slot:
            i = pending.pop(0)
            slots.admit(prompts[i], max_new_tokens=mnt[i], meta=i)
        for meta, r in slots.step():
            results[meta] = r
        rounds += 1
        assert rounds < 200
    assert sorted(results) == list(range(len(prompts)))
    for i, p in enumerate(prompts):
        assert results[i].num_tokens >= mnt[i]
        _check_greedy(target.model, p, results[i].token_ids)
    with pytest.raises(RuntimeError):
        full = SpecSlots(target, tok, d, capacity=1, max_ctx=128)
        full.admit(prompts[0], max_new_tokens=2)
        full.admit(prompts[1], max_new_tokens=2)


def test_shared_prefix_pages_are_token_identical(dev, pair):
    """Rows whose prompts start with a registered prefix read its K/V (and the drafter's
    context) from shared pages; the outputs equal those of private prefills exactly."""
    from mlx_dspark.batch_engine import SpecSlots
    target, tok, d, cfg = pair
    V = target.model.args.vocab_size
    prefix = _prompts(V, [128], 3)[0]
    suffixes = _prompts(V, [5, 19, 11], 4)
    prompts = [prefix + s for s in suffixes]

    def run(share):
        slots = SpecSlots(target, tok, d, capacity=3, max_draft_tokens=3, max_ctx=320, prefix_pages=4 if share else 0)
        if share:
            assert slots.register_prefix(prefix) == 128
        for i, p in enumerate(prompts):
            slots.admit(p, max_new_tokens=12, meta=i)
        out = {}
        while slots.n_active:
            for meta, r in slots.step():
                out[meta] = r.token_ids
        return [out[i] for i in range(len(prompts))]

    shared, private = run(True), run(False)
    assert shared == private
    for p, t in zip(prompts, shared):
        _check_greedy(target.model, p, t)


def test_batch_generate_baseline_rows_follow_greedy(dev, pair):
    from mlx_dspark.batch_engine import batch_generate_baseline
    target, tok, d, cfg = pair
    prompts = _prompts(target.model.args.vocab_size, [12, 30], 9)
    res = batch_generate_baseline(target, tok, prompts, max_new_tokens=[10, 7])
    assert [r.num_tokens for r in res] == [10, 7]
    for p, r in zip(prompts, res):
        _check_greedy(target.model, p, r.token_ids)


def test_spec_slots_sampled_is_seeded(dev, pair):
    from mlx_dspark.batch_engine import batch_spec_generate
    target, tok, d, cfg = pair
    prompts = _prompts(target.model.args.vocab_size, [15, 26], 5)
    kw = dict(max_new_tokens=14, max_draft_tokens=3, temperature=0.7, top_k=50)
    a = batch_spec_generate(target, tok, d, prompts, seed=42, **kw)
    b = batch_spec_generate(target, tok, d, prompts, seed=42, **kw)
    c = batch_spec_generate(target, tok, d, prompts, seed=43, **kw)
    assert [r.token_ids for r in a] == [r.token_ids for r in b]
    assert [r.token_ids for r in a] != [r.token_ids for r in c]
    for r in a:
        assert sum(r.accept_lengths) + 1 == r.num_tokens
        assert all(0 <= t < target.model.args.vocab_size for t in r.token_ids)
