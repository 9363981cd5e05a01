"""CPU checks of the DSpark host logic and oracle against the reference's own test vectors:
Markov block sampling control flow (tests/test_batch_engine.py:214-238), presence/frequency
penalty rows (tests/test_penalties.py:14-57), the n-gram lookup index (tests/test_lookup.py),
drafter config parsing (tests/test_formats.py:26-107 fixtures), and the oracle's Markov step
against a brute-force loop."""

import json

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import w8 as W8

# ------------------------------------------------------------------ Markov block sampling


def test_markov_no_head_is_rowwise_argmax():
    # tests/test_batch_engine.py:214-225: base one-hot rows -> [[2, 4, 1], [0, 3, 2]]
    base = torch.zeros((2, 3, 5))
    for (r, c, v) in [(0, 0, 2), (0, 1, 4), (0, 2, 1), (1, 0, 0), (1, 1, 3), (1, 2, 2)]:
        base[r, c, v] = 1.0
    got = [OM.markov_sample_block(base[b], 9, lambda p: torch.zeros(5)) for b in range(2)]
    assert got == [[2, 4, 1], [0, 3, 2]]


def test_markov_chain_follows_previous_token():
    # tests/test_batch_engine.py:228-238: bias strongly favours prev + 1 -> [[1, 2], [3, 4]]
    def step_bias(prev):
        return (torch.arange(5) == (prev + 1) % 5).float() * 100.0
    got = [OM.markov_sample_block(torch.zeros((2, 5)), p, step_bias) for p in (0, 2)]
    assert got == [[1, 2], [3, 4]]


def test_oracle_markov_step_matches_bruteforce():
    rng = np.random.default_rng(0)
    V, R = 64, 256
    w1 = (rng.standard_normal((V, R)) * 0.1).astype(np.float32)
    w2 = (rng.standard_normal((V, R)) * 0.1).astype(np.float32)
    q1, s1, b1 = W8.quantize(w1)
    q2, s2, b2 = W8.quantize(w2)

    class D:
        pass
    o = OM.OracleDSpark.__new__(OM.OracleDSpark)
    o.w1 = torch.from_numpy(W8.dequantize(q1, s1, b1).astype(np.float32))
    o.w2 = torch.from_numpy(W8.dequantize(q2, s2, b2).astype(np.float32))
    base = torch.from_numpy(rng.standard_normal((3, V)).astype(np.float32))
    toks = o.sample_block(base, 7)
    prev = 7
    d1, d2 = W8.dequantize(q1, s1, b1), W8.dequantize(q2, s2, b2)
    for i in range(3):
        e = W8.bf16_round(d1[prev].astype(np.float32)).astype(np.float64)
        bias = np.array([sum(d2[v, r] * e[r] for r in range(R)) for v in range(V)])
        row = W8.bf16_round(W8.bf16_round(base[i].numpy()) + W8.bf16_round(bias.astype(np.float32)))
        assert toks[i] == int(np.argmax(row))            # numpy argmax: lowest index on ties
        prev = toks[i]


# ------------------------------------------------------------------ penalties

@pytest.fixture(params=["oracle", "engine"])
def rows_fn(request):
    if request.param == "oracle":
        return lambda counts, pres, freq, prefix: OM.penalty_rows(counts, pres, freq, prefix)
    from mlx_dspark.generate import _Penalizer

    def f(counts, pres, freq, prefix):
        p = _Penalizer(pres, freq)
        p.counts = dict(counts)
        return p.block_rows(prefix)
    return f


def test_penalty_base_presence_and_frequency(rows_fn):
    # tests/test_penalties.py:21-31: counts {5: 2, 2: 1}, presence 1, frequency 0.5
    rows = rows_fn({5: 2, 2: 1}, 1.0, 0.5, [])
    assert len(rows) == 1
    assert abs(rows[0][5] - 2.0) < 1e-9 and abs(rows[0][2] - 1.5) < 1e-9
    assert rows[0].get(0, 0.0) == 0.0 and rows[0].get(3, 0.0) == 0.0


def test_penalty_draft_prefix_new_token(rows_fn):
    # tests/test_penalties.py:34-41: prefix [3, 3] -> column 3 = 0, 1.5, 2.0
    rows = rows_fn({}, 1.0, 0.5, [3, 3])
    assert [r.get(3, 0.0) for r in rows] == [0.0, 1.5, 2.0]


def test_penalty_draft_prefix_token_in_base(rows_fn):
    # tests/test_penalties.py:44-50: base {7: 1}, prefix [7] -> 1.5, 2.0
    rows = rows_fn({7: 1}, 1.0, 0.5, [7])
    assert [r.get(7, 0.0) for r in rows] == [1.5, 2.0]


def test_penalty_apply_rows(rows_fn):
    # tests/test_penalties.py:53-57: presence 2, base {1}, prefix [3]
    rows = rows_fn({1: 1}, 2.0, 0.0, [3])
    out = np.zeros((2, 4))
    for i, r in enumerate(rows):
        for t, v in r.items():
            out[i, t] -= v
    assert out.tolist() == [[0.0, -2.0, 0.0, 0.0], [0.0, -2.0, 0.0, -2.0]]


# ------------------------------------------------------------------ n-gram lookup (tests/test_lookup.py)

def _idx(tokens, **kw):
    from mlx_dspark.lookup import NGramIndex
    ix = NGramIndex(**kw)
    ix.extend(list(tokens))
    return ix


def test_lookup_vectors():
    assert _idx([5, 6, 7, 0, 1, 2, 5, 6]).propose() == []
    assert _idx([4, 5, 6, 7, 8, 0, 4, 5, 6], max_draft=2).propose() == [7, 8]
    assert _idx([1, 2, 3, 4]).propose() == []
    assert _idx([5, 6, 7, 8, 9, 1, 5, 6], min_n=2, max_n=3, max_draft=3).propose() == [7, 8, 9]
    assert _idx([1, 2, 3, 4, 5], min_n=2, max_n=3).propose() == []
    assert _idx([5, 6, 7, 0, 5, 6, 8, 0, 5, 6], min_n=2, max_n=3, max_draft=1).propose() == [8]
    assert _idx([4, 5, 6, 9, 0, 5, 6, 7, 0, 4, 5, 6], min_n=2, max_n=3, max_draft=1).propose() == [9]
    assert _idx([5, 6, 7, 8, 9, 10, 11, 0, 5, 6], min_n=2, max_n=3, max_draft=4).propose() == [7, 8, 9, 10]
    assert _idx([1, 9, 9, 2, 9, 9], min_n=2, max_n=3, max_draft=4).propose() == [2, 9, 9]


def test_lookup_incremental_matches_bulk():
    from mlx_dspark.lookup import NGramIndex
    toks = [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 9]
    bulk = _idx(toks, min_n=2, max_n=3, max_draft=2)
    inc = NGramIndex(min_n=2, max_n=3, max_draft=2)
    for t in toks:
        inc.extend([t])
    assert bulk.propose() == inc.propose()


# ------------------------------------------------------------------ config parsing (tests/test_formats.py fixtures)

QWEN3_MIN = {"model_type": "qwen3", "hidden_size": 16, "vocab_size": 32, "num_hidden_layers": 1,
             "intermediate_size": 32, "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 8,
             "block_size": 4, "mask_token_id": 3, "target_layer_ids": [0, 1], "num_target_layers": 2,
             "markov_rank": 4}
GEMMA4_MIN = {"model_type": "gemma4_text", "hidden_size": 16, "vocab_size": 32, "num_hidden_layers": 1,
              "intermediate_size": 32, "num_attention_heads": 2, "num_key_value_heads": 1,
              "num_global_key_value_heads": 1, "head_dim": 8, "global_head_dim": 8, "block_size": 4,
              "mask_token_id": 3, "target_layer_ids": [0, 1], "num_target_layers": 2, "markov_rank": 4}
SPECULATORS = {"architectures": ["DSparkDraftModel"], "model_type": "qwen3", "speculators_model_type": "dspark",
               "speculators_config": {"algorithm": "dspark"}, "block_size": 8, "markov_rank": 256}
EMBEDDED_V4 = {"model_type": "deepseek_v4", "hidden_size": 7168, "num_hidden_layers": 61, "vocab_size": 129280,
               "dspark_block_size": 5, "dspark_target_layer_ids": [58, 59, 60], "dspark_markov_rank": 512}


def _cfg(tmp_path, c):
    from mlx_dspark.config import DSparkConfig
    p = tmp_path / "config.json"
    p.write_text(json.dumps(c))
    return DSparkConfig.from_json(p)


def test_config_parsing(tmp_path):
    c = _cfg(tmp_path, QWEN3_MIN)
    assert c.family == "qwen3" and c.block_size == 4 and c.norm_style == "qwen" and c.mlp_activation == "silu"
    assert c.scaling == 8 ** -0.5 and c.n_kv_heads == 1 and not c.use_v_norm
    g = _cfg(tmp_path, GEMMA4_MIN)
    assert g.family == "gemma4" and g.target_layer_ids == [0, 1] and g.scaling == 1.0 and g.n_kv_heads == 1
    with pytest.raises(ValueError, match="speculators"):
        _cfg(tmp_path, SPECULATORS)
    with pytest.raises(ValueError, match="embedded"):
        _cfg(tmp_path, EMBEDDED_V4)
    with pytest.raises(ValueError, match="unsupported drafter family"):
        _cfg(tmp_path, {**QWEN3_MIN, "model_type": "llama"})
    with pytest.raises(ValueError, match="unsupported drafter family"):
        _cfg(tmp_path, {k: v for k, v in QWEN3_MIN.items() if k != "model_type"})
    with pytest.raises(ValueError, match="target_layer_ids"):
        _cfg(tmp_path, {k: v for k, v in QWEN3_MIN.items() if k != "target_layer_ids"})


def test_proportional_rope_frequencies_match_transformers():
    """The oracle's proportional RoPE table (gemma4 drafter) against transformers' published
    definition (_compute_proportional_rope_parameters), and the engine's table against the
    oracle's: the first int(0.25 * hd / 2) frequencies are theta^(-2i/hd), the rest 0."""
    from transformers import PretrainedConfig
    from transformers import modeling_rope_utils as m
    for hd, frac, theta in ((512, 0.25, 1e6), (256, 0.5, 1e4), (128, 1.0, 1e6)):
        cfg = PretrainedConfig(head_dim=hd, hidden_size=hd * 4, num_attention_heads=4,
                               rope_parameters={"rope_type": "proportional", "rope_theta": theta,
                                                "partial_rotary_factor": frac})
        want, _ = m.ROPE_INIT_FUNCTIONS["proportional"](cfg, "cpu")
        got = OM.inv_freq(hd, theta, frac)
        assert got.shape == want.shape
        assert torch.allclose(got, want.float(), rtol=2e-6, atol=0), (hd, frac)
        n_rot = int(frac * hd // 2)
        assert torch.all(got[n_rot:] == 0) and torch.all(got[:n_rot] > 0)
        from mlx_dspark.ops import rope_inv_freq
        assert torch.equal(rope_inv_freq(hd, theta, "cpu", rotary_fraction=frac), got)


def test_proportional_rope_leaves_unrotated_dims():
    """Dims whose frequency is 0 pass through RoPE unchanged (closed form); the rotated ones
    keep their pair norms."""
    hd = 512
    inv = OM.inv_freq(hd, 1e6, 0.25)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 5, hd, generator=g)
    pos = torch.tensor([0, 7, 100, 4095, 8191])
    y = OM.rope(x, pos, 1e6, inv)
    n_rot = 64
    keep = torch.cat([torch.arange(n_rot, hd // 2), torch.arange(hd // 2 + n_rot, hd)])
    assert torch.equal(y[..., keep], x[..., keep])
    r_in = x[..., :n_rot] ** 2 + x[..., hd // 2:hd // 2 + n_rot] ** 2
    r_out = y[..., :n_rot] ** 2 + y[..., hd // 2:hd // 2 + n_rot] ** 2
    assert torch.allclose(r_in, r_out, rtol=1e-5)
    assert torch.equal(y[:, 0], x[:, 0])       # position 0: identity


# ------------------------------------------------------------------ confidence head


@pytest.mark.parametrize("with_markov", [True, False])
def test_confidence_logits_one_hot_projection(with_markov):
    """OracleDSpark.confidence_logits against what the mathematics fixes. The reference's head
    is proj(features) with nn.Linear's bias (src/mlx_dspark/model.py:211-217), the features the
    block hidden rows followed by w1[prev] when config.confidence_head_with_markov (:311-320).
    With a projection whose codes make it exactly the unit vector e_i (q = 1 at i, scale 1,
    bias 0: dequantized exactly), the logit of row r is h[r, i] + b for i < H and
    bf16(w1[prev_r])[i - H] + b past H; e_i past H does not exist without the Markov features.
    Catches a swapped concat order, a missing or doubled bias, a Markov row taken at another
    token and the concat keyed on anything but the config flag."""
    import dataclasses
    import types
    from _oracle_models import _dspark, _table

    g = torch.Generator().manual_seed(3)
    H, V, R = 64, 96, 64
    d = _dspark(g, "qwen3", H, 128, V, 1e-6, False)
    d.config = dataclasses.replace(d.config, markov_rank=R, confidence_head_with_markov=with_markov)
    w1 = _table(0.3 * torch.randn(V, R, generator=g))
    d.markov_head = types.SimpleNamespace(w1=w1, w2=types.SimpleNamespace(mlx=w1.mlx))
    K = H + (R if with_markov else 0)
    bias = 0.375
    rows = torch.randn(5, H, generator=g)
    prev = torch.tensor([3, 17, 17, 95, 0])
    w1f = OM.bf(OM.deq_table(w1))
    for i in list(range(0, H, 7)) + ([H, H + 1, H + 33, K - 1] if with_markov else [H - 1]):
        q = torch.zeros(16, K, dtype=torch.uint8)
        q[0, i] = 1
        s = torch.ones(16, K // 64, dtype=torch.bfloat16)
        b = torch.zeros(16, K // 64, dtype=torch.bfloat16)
        d.confidence_head = types.SimpleNamespace(proj=types.SimpleNamespace(mlx=(q, s, b)), bias=bias)
        o = OM.OracleDSpark(d)
        got = o.confidence_logits(rows, prev)
        want = rows[:, i] + bias if i < H else w1f[prev, i - H] + bias
        assert torch.equal(got, want), i
