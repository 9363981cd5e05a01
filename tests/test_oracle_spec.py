"""CPU pins of the oracle's speculative loops (oracle/spec.py): greedy speculative decoding
reproduces plain greedy decoding token for token whatever the drafter proposes, so both loops
must equal model.greedy_decode on the same weights; a drafter that is always right must be
accepted whole every round and one that is always wrong must commit one token per round."""

import types

import pytest
import torch

from _oracle_models import _dspark, _layer, _norm_w, _target, _wobj
from oracle import model as OM
from oracle import spec as SP

N_NEW = 14


@pytest.fixture(autouse=True)
def no_rounding(monkeypatch):
    """float32 throughout: forwards of different widths then agree far below any pick margin."""
    monkeypatch.setattr(OM, "bf", lambda x: x)


def _models(seed):
    from mlx_dspark.qwen3 import TargetArgs
    g = torch.Generator().manual_seed(seed)
    a = TargetArgs(model_type="qwen3", hidden_size=128, num_hidden_layers=3, intermediate_size=256,
                   num_attention_heads=4, num_key_value_heads=2, head_dim=32, vocab_size=300)
    m = _target(a, g)
    prompt = torch.randint(0, a.vocab_size, (11,), generator=g).tolist()
    return a, m, g, prompt


def _greedy(m, prompt):
    return OM.greedy_decode(OM.OracleTarget(m), prompt, N_NEW)[0]


@pytest.mark.parametrize("mode", ["drafter", "right", "wrong"])
def test_dspark_loop_is_greedy_decoding(mode, monkeypatch):
    a, m, g, prompt = _models(1)
    want = _greedy(m, prompt)
    d = _dspark(g, "qwen3", a.hidden_size, a.intermediate_size, a.vocab_size, 1e-6, False)
    d.config.block_size = 5
    od = OM.OracleDSpark(d)
    cap = 4
    if mode != "drafter":            # drafts from the known greedy stream, right or shifted
        stream = want + [0] * 8
        pos = {"i": 0}

        def planted(base, first_prev):
            i = want.index(first_prev, pos["i"]) if first_prev in want[pos["i"]:] else pos["i"]
            pos["i"] = i
            picks = stream[i + 1:i + 1 + cap]
            return picks if mode == "right" else [(t + 1) % a.vocab_size for t in picks]

        monkeypatch.setattr(od, "sample_block", planted)
    got, accepts = SP.dspark_generate(OM.OracleTarget(m), od, prompt, N_NEW, cap, (0, 2), a.vocab_size - 1, 5)
    assert got[:N_NEW] == want
    if mode == "right":
        assert all(n == cap + 1 for n in accepts[:-1])
    if mode == "wrong":
        assert all(n == 1 for n in accepts)


def test_dflash_loop_is_greedy_decoding():
    a, m, g, prompt = _models(2)
    want = _greedy(m, prompt)
    H, I = a.hidden_size, a.intermediate_size
    c = types.SimpleNamespace(num_attention_heads=4, num_key_value_heads=2, head_dim=32, rms_norm_eps=1e-6,
                              rope_theta=1e6, layer_types=("sliding_attention", "full_attention"),
                              sliding_window=6)
    drafter = types.SimpleNamespace(config=c, fc=_wobj(0.05 * torch.randn(H, 2 * H, generator=g)),
                                    hidden_norm=_norm_w(H, g), norm=_norm_w(H, g),
                                    layers=[_layer(g, H, I, 4, 2, 32) for _ in range(2)])
    tgt = OM.OracleTarget(m)
    od = OM.OracleDFlash(drafter, tgt)
    got, accepts = SP.dflash_generate(tgt, od, prompt, N_NEW, 5, (0, 2), a.vocab_size - 1, 6)
    assert got[:N_NEW] == want
    assert sum(accepts) + 1 == len(got)
    # one drafter context row per committed position, the last round's rows still to come
    assert od.offset == tgt.offset - accepts[-1]


def test_greedy_accept_counts_the_matching_prefix():
    assert SP.greedy_accept([3, 4, 5, 6], [3, 4, 9]) == 2
    assert SP.greedy_accept([3, 4, 5, 6], [3, 4, 5]) == 3
    assert SP.greedy_accept([1], []) == 0
    assert SP.greedy_accept([2, 2], [1]) == 0
