"""GPU: the reference's own callers' call sequences, replayed against this package.

- The server's single-request path (src/mlx_dspark/server.py:143-158 and :272-329): the prefix
  store is built from the bound ``target.make_cache`` / ``drafter.make_ctx_cache`` as the
  server builds it, then every request runs acquire -> the mode's generate function with the
  keyword arguments the server passes -> store (reset when the generation raises). Two turns
  per mode; turn 2 reuses turn 1's KV where the mode allows it.
- The server's continuous-batching session (server.py:505-563): SpecSlots built with the
  server's arguments, admission while slots are free, mid-flight arrivals pulled into freed
  slots, and each result delivered as its row retires.

Greedy streams are checked against the oracle's greedy decoding (tests/_parity.py)."""

import numpy as np
import pytest

from _parity import check_greedy_stream

pytestmark = pytest.mark.gpu
MIN_MATCH = 8


@pytest.fixture(scope="module")
def models(dev):
    from mlx_dspark.load import load_dflash_pair, load_pair
    target, tok, d, _ = load_pair("synthetic/tiny", keep_mlx=True)
    t2, tok2, dfl, _ = load_dflash_pair("synthetic/tiny", keep_mlx=True)
    return {"dspark": (target, tok, d), "dflash": (t2, tok2, dfl)}


def _build_prefix(mode, target, drafter, slots=2, l2_dir=None, max_ram_mb=0):
    from mlx_dspark.prefix_cache import PrefixCache, target_cache_reusable
    if mode == "dflash" or not target_cache_reusable(target.make_cache(max_ctx=64)):
        return None
    make_ctx = drafter.make_ctx_cache if mode == "dspark" else None
    return PrefixCache(target.make_cache, make_ctx, l2_dir=l2_dir, max_ram_bytes=max(0, max_ram_mb) * 1024 * 1024,
                       slots=slots)


def _generate_impl(mode, prefix, target, tok, drafter, prompt_ids, max_tokens, temperature, top_p, top_k, stop,
                   seed, on_text, presence_penalty=0.0, frequency_penalty=0.0, logprobs=None,
                   max_draft_tokens=None, cap_controller=None, lookup_drafts=True, confidence_threshold=0.0):
    from mlx_dspark.generate import dflash_generate, greedy_generate, speculative_generate
    from mlx_dspark.lookup import lookup_generate
    cache = ctx = None
    reuse_len = 0
    if prefix is not None:
        cache, ctx, reuse_len = prefix.acquire(prompt_ids)
    try:
        if mode == "dspark":
            res = speculative_generate(
                target, tok, drafter, prompt_ids=prompt_ids, cache=cache, ctx_caches=ctx, reuse_len=reuse_len,
                max_new_tokens=max_tokens, max_draft_tokens=max_draft_tokens, cap_controller=cap_controller,
                lookup_drafts=lookup_drafts, confidence_threshold=confidence_threshold, temperature=temperature,
                top_p=top_p, top_k=top_k, presence_penalty=presence_penalty, frequency_penalty=frequency_penalty,
                logprobs=logprobs, seed=seed, stop=stop, on_text=on_text)
        elif mode == "dflash":
            res = dflash_generate(
                target, tok, drafter, prompt_ids=prompt_ids, max_new_tokens=max_tokens,
                max_draft_tokens=max_draft_tokens, cap_controller=cap_controller, temperature=temperature,
                top_p=top_p, top_k=top_k, seed=seed, stop=stop, on_text=on_text)
        elif mode == "lookup":
            res = lookup_generate(
                target, tok, prompt_ids=prompt_ids, cache=cache, reuse_len=reuse_len, max_new_tokens=max_tokens,
                max_draft_tokens=max_draft_tokens or 6, temperature=temperature, top_p=top_p, top_k=top_k,
                seed=seed, stop=stop, on_text=on_text)
        else:
            res = greedy_generate(
                target, tok, prompt_ids=prompt_ids, cache=cache, reuse_len=reuse_len, max_new_tokens=max_tokens,
                temperature=temperature, top_p=top_p, top_k=top_k, presence_penalty=presence_penalty,
                frequency_penalty=frequency_penalty, logprobs=logprobs, seed=seed, stop=stop, on_text=on_text)
    except BaseException:
        if prefix is not None:
            prefix.reset()
        raise
    if prefix is not None and cache is not None:
        prefix.store(cache, ctx, prompt_ids, res.token_ids)
    return res


@pytest.mark.parametrize("mode", ["dspark", "baseline", "lookup", "dflash"])
def test_server_single_request_sequence(dev, models, mode):
    target, tok, d = models["dflash" if mode == "dflash" else "dspark"]
    print(f"server sequence mode={mode}", flush=True)
    prefix = _build_prefix(mode, target, d)
    mdt = {"dspark": 2, "lookup": 6}.get(mode)
    V = target.model.args.vocab_size
    rng = np.random.default_rng(31)
    t1 = rng.integers(0, V, 48).tolist()
    r1 = _generate_impl(mode, prefix, target, tok, d, t1, 16, 0.0, 1.0, 0, None, None, None, max_draft_tokens=mdt)
    t2 = t1 + r1.token_ids + rng.integers(0, V, 10).tolist()
    r2 = _generate_impl(mode, prefix, target, tok, d, t2, 16, 0.0, 1.0, 0, None, None, None, max_draft_tokens=mdt)
    for prompt, res in ((t1, r1), (t2, r2)):
        assert 16 <= res.num_tokens <= 16 + (mdt or 0)     # lookup commits whole rounds
        check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    if mode == "dflash":
        assert prefix is None
    else:
        info = prefix.info()
        assert info["hits"] == 1 and info["reused_tokens"] == len(t1) + len(r1.token_ids) - 1
        assert len(info["slots"]) == 1 and info["slots"][0]["tokens"] == len(t2) + 15


def test_server_resets_the_prefix_store_when_a_generation_raises(dev, models):
    target, tok, d = models["dspark"]
    prefix = _build_prefix("dspark", target, d)
    V = target.model.args.vocab_size
    t1 = np.random.default_rng(5).integers(0, V, 40).tolist()
    _generate_impl("dspark", prefix, target, tok, d, t1, 8, 0.0, 1.0, 0, None, None, None, max_draft_tokens=2)
    assert len(prefix.info()["slots"]) == 1

    def boom(text):
        raise KeyboardInterrupt

    with pytest.raises(KeyboardInterrupt):
        _generate_impl("dspark", prefix, target, tok, d, t1 + [1, 2], 8, 0.0, 1.0, 0, None, None, boom,
                       max_draft_tokens=2)
    assert prefix.info()["slots"] == []
    res = _generate_impl("dspark", prefix, target, tok, d, t1, 8, 0.0, 1.0, 0, None, None, None, max_draft_tokens=2)
    check_greedy_stream(target.model, t1, res.token_ids, MIN_MATCH)


def test_server_batching_session_sequence(dev, models):
    from mlx_dspark.batch_engine import SpecSlots
    target, tok, d = models["dspark"]
    V = target.model.args.vocab_size
    rng = np.random.default_rng(41)
    jobs = [{"id": i, "prompt_ids": rng.integers(0, V, int(n)).tolist(), "max_tokens": int(m)}
            for i, (n, m) in enumerate([(40, 10), (70, 24), (33, 6), (52, 16), (45, 12), (61, 8)])]
    arrivals = jobs[3:]                                   # come in while the session runs
    max_batch = 3
    slots = SpecSlots(target, tok, d, capacity=max_batch, max_draft_tokens=2, cap_controller=None)
    waiting = list(jobs[:3])
    done, order, peak, steps = {}, [], 0, 0
    while slots.n_active or waiting or arrivals:
        while waiting and slots.has_free_slot:
            job = waiting.pop(0)
            slots.admit(job["prompt_ids"], max_new_tokens=job["max_tokens"], on_text=None, stop=None, meta=job)
        while len(waiting) < max_batch and arrivals and steps % 2 == 1:
            waiting.append(arrivals.pop(0))
        while waiting and slots.has_free_slot:
            job = waiting.pop(0)
            slots.admit(job["prompt_ids"], max_new_tokens=job["max_tokens"], on_text=None, stop=None, meta=job)
        peak = max(peak, slots.n_active)
        for job, res in slots.step():
            done[job["id"]] = res
            order.append((job["id"], steps))
        steps += 1
    assert sorted(done) == list(range(len(jobs))) and peak == max_batch
    assert order[0][1] < order[-1][1]                     # rows retire as they finish
    for job in jobs:
        res = done[job["id"]]
        # a round commits up to cap + 1 tokens, so a row may end past its limit (as in the reference)
        assert job["max_tokens"] <= res.num_tokens <= job["max_tokens"] + 2
        check_greedy_stream(target.model, job["prompt_ids"], res.token_ids, min(MIN_MATCH, job["max_tokens"]))
