"""GPU: a second conversation turn served from the prefix KV cache (the server's
acquire -> generate -> store flow, src/mlx_dspark/server.py:276-320) decodes the same greedy
stream as the oracle's cold decode of the whole prompt (to the top-2 margin rule), with DSpark
speculative decoding and with plain greedy decoding, from HBM slots and from spilled ones."""

import functools

import numpy as np
import pytest

from _parity import check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2          # greedy-stream margin rule (normalised logits)


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


def _check_greedy(target, prompt, got):
    check_greedy_stream(target.model, prompt, got, MIN_MATCH)


@pytest.mark.parametrize("mode,spill", [("dspark", False), ("dspark", True), ("greedy", False)])
def test_second_turn_reuses_the_first(dev, pair, tmp_path, mode, spill):
    from mlx_dspark.generate import greedy_generate, speculative_generate
    from mlx_dspark.prefix_cache import PrefixCache
    target, tok, d, cfg = pair
    print(f"prefix cache mode={mode} spill={spill}", flush=True)
    max_ctx = 512
    pc = PrefixCache(functools.partial(target.make_cache, max_ctx=max_ctx),
                     functools.partial(d.make_ctx_cache, max_ctx=max_ctx) if mode == "dspark" else None,
                     min_reuse=8, l2_dir=str(tmp_path) if spill else None, max_ram_bytes=1 if spill else 0)

    def serve(ids):
        cache, ctx, reuse = pc.acquire(ids)
        if mode == "dspark":
            res = speculative_generate(target, tok, d, prompt_ids=ids, cache=cache, ctx_caches=ctx, reuse_len=reuse,
                                       max_new_tokens=20, max_draft_tokens=None)
        else:
            res = greedy_generate(target, tok, prompt_ids=ids, cache=cache, reuse_len=reuse, max_new_tokens=20)
        pc.store(cache, ctx, ids, res.token_ids)
        return res, reuse

    rng = np.random.default_rng(21)
    turn1 = rng.integers(0, target.model.args.vocab_size, 60).tolist()
    res1, reuse1 = serve(turn1)
    assert reuse1 == 0
    if spill:
        assert pc.info()["slots"][0]["spilled"]
    turn2 = turn1 + res1.token_ids + rng.integers(0, target.model.args.vocab_size, 12).tolist()
    res2, reuse2 = serve(turn2)
    assert reuse2 == len(turn1) + len(res1.token_ids) - 1
    assert pc.info()["hits"] == 1
    _check_greedy(target, turn2, res2.token_ids)


def test_conversations_share_system_prompt_pages(dev, pair):
    """Two conversations with one system prompt: the second maps the first's whole pages of it
    (no copy) and both continue with the oracle's greedy streams; a third turn of the first
    conversation still finds its own pages."""
    from mlx_dspark.generate import speculative_generate
    from mlx_dspark.prefix_cache import PrefixCache
    target, tok, d, cfg = pair
    pc = PrefixCache(functools.partial(target.make_cache, max_ctx=512),
                     functools.partial(d.make_ctx_cache, max_ctx=512), min_reuse=8, slots=3)

    def serve(ids):
        cache, ctx, reuse = pc.acquire(ids)
        res = speculative_generate(target, tok, d, prompt_ids=ids, cache=cache, ctx_caches=ctx, reuse_len=reuse,
                                   max_new_tokens=16, max_draft_tokens=3)
        pc.store(cache, ctx, ids, res.token_ids)
        _check_greedy(target, ids, res.token_ids)
        return res, reuse

    V = target.model.args.vocab_size
    rng = np.random.default_rng(8)
    system = rng.integers(0, V, 150).tolist()            # 2 whole pages + 22 tokens
    a = system + rng.integers(0, V, 20).tolist()
    b = system + rng.integers(0, V, 31).tolist()
    ra, reuse_a = serve(a)
    rb, reuse_b = serve(b)
    assert reuse_a == 0 and reuse_b == 150
    assert pc.info()["pages"]["shared"] == 1 and len(pc.info()["slots"]) == 2
    a2 = a + ra.token_ids + rng.integers(0, V, 5).tolist()
    _, reuse_a2 = serve(a2)
    assert reuse_a2 == len(a) + len(ra.token_ids) - 1
