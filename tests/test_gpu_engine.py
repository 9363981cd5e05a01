"""GPU: the server-facing engine (src/mlx_dspark/server.py:75-370) serves a two-turn
conversation in every mode; turn 2 reuses turn 1's KV where the mode allows it, and the greedy
streams equal the oracle's cold greedy decoding (top-2 margin rule)."""

import numpy as np
import pytest

from oracle import model as OM

pytestmark = pytest.mark.gpu
TOL = 2e-2          # greedy-stream margin rule (normalised logits)


def _check_greedy(target, prompt, got):
    ref, margins = OM.greedy_decode(OM.OracleTarget(target.model), prompt, len(got))
    for i, (a, b) in enumerate(zip(got, ref)):
        if a != b:
            assert margins[i] <= TOL, (i, a, b, margins[i])
            break


@pytest.mark.parametrize("mode", ["dspark", "baseline", "lookup", "dflash"])
def test_engine_two_turns(dev, mode):
    from mlx_dspark.engine import Engine
    from mlx_dspark.load import load_dflash_pair, load_pair, load_target
    print(f"engine mode={mode}", flush=True)
    d = None
    if mode == "dspark":
        target, tok, d, _ = load_pair("synthetic/tiny", keep_mlx=True)      # the oracle reads MLX triplets
    elif mode == "dflash":
        target, tok, d, _ = load_dflash_pair("synthetic/tiny", keep_mlx=True)
    else:
        target, tok = load_target("synthetic/tiny", keep_mlx=True)
    eng = Engine(target, tok, d, mode=mode, model_id="tiny", max_ctx=1024,
                 max_draft_tokens={"dspark": 2, "lookup": 6}.get(mode))
    try:
        V = eng.target.model.args.vocab_size
        rng = np.random.default_rng(31)
        t1 = rng.integers(0, V, 48).tolist()
        r1 = eng.generate(t1, max_tokens=16, temperature=0.0, stop=None, seed=None)
        t2 = t1 + r1.token_ids + rng.integers(0, V, 10).tolist()
        r2 = eng.generate(t2, max_tokens=16, temperature=0.0, stop=None, seed=None)
        for prompt, res in ((t1, r1), (t2, r2)):
            assert res.num_tokens >= 1
            _check_greedy(eng.target, prompt, res.token_ids)
        m = eng.metrics()
        assert m["requests"] == 2 and m["completion_tokens"] == r1.num_tokens + r2.num_tokens
        if mode == "dflash":
            assert m["prefix_cache"] == {"enabled": False}
        else:
            assert m["prefix_cache"]["hits"] == 1
            assert m["prefix_cache"]["reused_tokens"] == len(t1) + len(r1.token_ids) - 1
        info = eng.spec_info(r2)
        assert info["mode"] == mode and info["target_forwards"] >= 1
    finally:
        eng.close()


def test_engine_load_by_name(dev):
    from mlx_dspark.engine import Engine
    eng = Engine.load(mode="dspark", model="synthetic/tiny", max_ctx=512)
    try:
        assert eng.max_draft_tokens == 2 and eng.prefix is not None
        res = eng.generate(list(range(40, 80)), max_tokens=8, temperature=0.0, stop=None, seed=None)
        assert res.num_tokens >= 1 and eng.metrics()["requests"] == 1
    finally:
        eng.close()
