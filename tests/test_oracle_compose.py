"""CPU pins of the oracle's layer compositions against independent implementations.

The verify forward (OracleTarget), the DFlash drafter (OracleDFlash) and the DSpark drafter
(OracleDSpark, both families) are compositions of norms, projections, RoPE, attention and MLPs
that the reference leaves to mlx_lm / mlx_vlm. Each is compared here, with the oracle's bf16
rounding points switched off, against the `transformers` implementation of the public
architecture on identical (dequantized) weights:
  - OracleTarget (qwen3) == Qwen3ForCausalLM: GQA, q/k RMSNorm, RoPE theta, untied and tied heads,
    a prompt then a KV-cached continuation, hidden-state taps;
  - OracleTarget (Gemma-style layout) == Gemma3ForCausalLM: sandwich norms, GeGLU, sliding-window
    layers with their own RoPE base (window shorter than the prompt), query_pre_attn_scalar, the
    final soft-cap, the sqrt(hidden) embedding scale;
  - OracleDFlash (src/mlx_dspark/dflash_model.py:100-208) == a stack of Qwen3DecoderLayer run
    without a mask over [context rows; block rows] at positions 0..S+L-1: with no context rows the
    drafter layer is exactly that stack; with context rows it is too when the context rows'
    input norm is the identity (unit weights, eps 0, rows of unit RMS, which hidden_norm with unit
    weights and eps 0 produces), so the context rows' K/V come from the same projections;
  - OracleDSpark qwen3 (src/mlx_dspark/model.py:83-262) == the same Qwen3DecoderLayer stack;
    OracleDSpark gemma4 == a stack of Gemma4TextDecoderLayer (k_eq_v with v_norm, proportional
    RoPE, scale 1, sandwich norms, layer_scalar).
Norm weights are random (not ones), so a misplaced or missing norm fails; each test also plants
one mistake (another RoPE base, a longer window, the block roped at the context's offset, a norm
weight left out) and checks that the comparison catches it.
"""

import types

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle import w8 as W8  # noqa: F401
from _oracle_models import _dspark, _layer, _norm_w, _target, _unit, _wobj  # noqa: F401

transformers = pytest.importorskip("transformers")
from transformers import Gemma3ForCausalLM, Gemma3TextConfig, Qwen3Config, Qwen3ForCausalLM  # noqa: E402
from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding  # noqa: E402

TOL = 1e-5   # normalized max-abs difference allowed between two float32 evaluations


@pytest.fixture(autouse=True)
def no_rounding(monkeypatch):
    """The oracle with every bf16 rounding point switched off (float32 throughout)."""
    monkeypatch.setattr(OM, "bf", lambda x: x)


def _attn_sd(L, nq, nkv, hd, shift=0.0):
    wq = OM.deq(L.qkv)
    return {"self_attn.q_proj.weight": wq[:nq * hd], "self_attn.k_proj.weight": wq[nq * hd:(nq + nkv) * hd],
            "self_attn.v_proj.weight": wq[(nq + nkv) * hd:], "self_attn.o_proj.weight": OM.deq(L.o),
            "self_attn.q_norm.weight": L.q_norm.float() - shift, "self_attn.k_norm.weight": L.k_norm.float() - shift}


def _mlp_sd(L, I):
    wgu = OM.deq(L.gate_up)
    return {"mlp.gate_proj.weight": wgu[:I], "mlp.up_proj.weight": wgu[I:], "mlp.down_proj.weight": OM.deq(L.down)}


# ------------------------------------------------------------------------------ verify forward
@pytest.mark.parametrize("tied", [False, True])
def test_target_qwen3_equals_transformers(tied):
    from mlx_dspark.qwen3 import TargetArgs
    g = torch.Generator().manual_seed(1 + tied)
    a = TargetArgs(model_type="qwen3", hidden_size=256, num_hidden_layers=3, intermediate_size=384,
                   num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=500, rope_theta=1e6,
                   tie_word_embeddings=tied)
    m = _target(a, g)
    H, I, nq, nkv, hd = a.hidden_size, a.intermediate_size, a.num_attention_heads, a.num_key_value_heads, a.head_dim
    cfg = Qwen3Config(hidden_size=H, num_hidden_layers=a.num_hidden_layers, intermediate_size=I, num_attention_heads=nq,
                      num_key_value_heads=nkv, head_dim=hd, vocab_size=a.vocab_size, rms_norm_eps=a.rms_norm_eps,
                      rope_theta=a.rope_theta, tie_word_embeddings=tied, attention_bias=False)
    cfg._attn_implementation = "eager"
    hf = Qwen3ForCausalLM(cfg).eval()
    sd = {"model.embed_tokens.weight": OM.deq_table(m.embed), "model.norm.weight": m.norm.float()}
    if not tied:
        sd["lm_head.weight"] = OM.deq(m.lm_head)
    for l, L in enumerate(m.layers):
        p = f"model.layers.{l}."
        sd.update({p + k: v for k, v in {**_attn_sd(L, nq, nkv, hd), **_mlp_sd(L, I)}.items()})
        sd[p + "input_layernorm.weight"] = L.in_norm.float()
        sd[p + "post_attention_layernorm.weight"] = L.post_norm.float()
    res = hf.load_state_dict(sd, strict=False)
    assert not res.unexpected_keys and set(res.missing_keys) <= {"lm_head.weight"}
    caps = {}
    for t in (0, 1):
        hf.model.layers[t].register_forward_hook(
            lambda mod, inp, out, t=t: caps.__setitem__(t, out[0] if isinstance(out, tuple) else out))
    ref = OM.OracleTarget(m)
    prompt = torch.randint(0, a.vocab_size, (7,), generator=g)
    block = torch.randint(0, a.vocab_size, (5,), generator=g)
    with torch.no_grad():
        o1 = hf(prompt[None], use_cache=True)
        l1, f1 = ref.forward(prompt, tap=(0, 1))
        assert OM.normalized_maxdiff(o1.logits[0], l1) < TOL
        assert torch.allclose(torch.cat([caps[0][0], caps[1][0]], -1), f1, atol=1e-5, rtol=1e-5)
        o2 = hf(block[None], past_key_values=o1.past_key_values, use_cache=True)
        l2, _ = ref.forward(block)
        assert OM.normalized_maxdiff(o2.logits[0], l2) < TOL
    # planted mistake in the oracle: another RoPE base changes the logits
    bad = OM.OracleTarget(types.SimpleNamespace(**{**m.__dict__, "args": TargetArgs(**{**a.__dict__, "rope_theta": 1e4})}))
    with torch.no_grad():
        assert OM.normalized_maxdiff(o1.logits[0], bad.forward(prompt)[0]) > 1e-3


def test_target_gemma_layout_equals_transformers():
    from mlx_dspark.qwen3 import TargetArgs
    g = torch.Generator().manual_seed(3)
    lt = tuple("full_attention" if (l + 1) % 6 == 0 else "sliding_attention" for l in range(6))
    a = TargetArgs(model_type="gemma3_text", hidden_size=256, num_hidden_layers=6, intermediate_size=384,
                   num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=500, rope_theta=1e6,
                   tie_word_embeddings=True, hidden_act="gelu_tanh", embed_scale=16.0, sliding_window=4,
                   layer_types=lt, final_logit_softcapping=30.0, query_pre_attn_scalar=48.0,
                   rope_local_base_freq=1e4)
    m = _target(a, g)
    H, I, nq, nkv, hd = a.hidden_size, a.intermediate_size, a.num_attention_heads, a.num_key_value_heads, a.head_dim
    cfg = Gemma3TextConfig(hidden_size=H, num_hidden_layers=6, intermediate_size=I, num_attention_heads=nq,
                           num_key_value_heads=nkv, head_dim=hd, vocab_size=a.vocab_size, rms_norm_eps=a.rms_norm_eps,
                           sliding_window=4, layer_types=list(lt), query_pre_attn_scalar=48,
                           final_logit_softcapping=30.0, attn_logit_softcapping=None,
                           hidden_activation="gelu_pytorch_tanh", tie_word_embeddings=True,
                           rope_parameters={"sliding_attention": {"rope_type": "default", "rope_theta": 1e4},
                                            "full_attention": {"rope_type": "default", "rope_theta": 1e6}})
    cfg._attn_implementation = "eager"
    hf = Gemma3ForCausalLM(cfg).eval()
    # gemma norms multiply by (1 + w); the oracle stores the effective multiplier
    sd = {"model.embed_tokens.weight": OM.deq_table(m.embed), "model.norm.weight": m.norm.float() - 1}
    for l, L in enumerate(m.layers):
        p = f"model.layers.{l}."
        sd.update({p + k: v for k, v in {**_attn_sd(L, nq, nkv, hd, shift=1.0), **_mlp_sd(L, I)}.items()})
        sd[p + "input_layernorm.weight"] = L.in_norm.float() - 1
        sd[p + "post_attention_layernorm.weight"] = L.attn_out_norm.float() - 1
        sd[p + "pre_feedforward_layernorm.weight"] = L.post_norm.float() - 1
        sd[p + "post_feedforward_layernorm.weight"] = L.ff_out_norm.float() - 1
    res = hf.load_state_dict(sd, strict=False)
    assert not res.unexpected_keys and set(res.missing_keys) <= {"lm_head.weight"}
    assert float(hf.model.embed_tokens.embed_scale) == a.embed_scale
    ref = OM.OracleTarget(m)
    prompt = torch.randint(0, a.vocab_size, (9,), generator=g)     # longer than the window of 4
    block = torch.randint(0, a.vocab_size, (5,), generator=g)
    with torch.no_grad():
        o1 = hf(prompt[None], use_cache=True)
        l1, _ = ref.forward(prompt)
        assert OM.normalized_maxdiff(o1.logits[0], l1) < TOL
        o2 = hf(block[None], past_key_values=o1.past_key_values, use_cache=True)
        l2, _ = ref.forward(block)
        assert OM.normalized_maxdiff(o2.logits[0], l2) < TOL
    # planted mistake in the oracle: a sliding window one token longer changes the logits
    ref2 = OM.OracleTarget(m)
    ref2.a = TargetArgs(**{**a.__dict__, "sliding_window": 5})
    with torch.no_grad():
        l1b, _ = ref2.forward(prompt)
    assert OM.normalized_maxdiff(o1.logits[0], l1b) > 1e-3


# ------------------------------------------------------------------------------ drafters
def _qwen3_stack(layers, H, I, nq, nkv, hd, eps, theta):
    cfg = Qwen3Config(hidden_size=H, num_hidden_layers=len(layers), intermediate_size=I, num_attention_heads=nq,
                      num_key_value_heads=nkv, head_dim=hd, vocab_size=16, rms_norm_eps=eps, rope_theta=theta)
    cfg._attn_implementation = "eager"
    out = []
    for l, L in enumerate(layers):
        d = Qwen3DecoderLayer(cfg, l).eval()
        d.load_state_dict({**_attn_sd(L, nq, nkv, hd), **_mlp_sd(L, I), "input_layernorm.weight": L.in_norm.float(),
                           "post_attention_layernorm.weight": L.post_norm.float()})
        out.append(d)
    return cfg, out


def _run_qwen3_stack(cfg, stack, ctx, h, shift=0, windows=None):
    """Each layer over [ctx; h] at positions 0.. (the block rows' positions moved by `shift`):
    without a mask, or, where windows[l] > 0, causal with that window (an additive mask); the
    block rows carry on, the context rows restart every layer."""
    rot = Qwen3RotaryEmbedding(cfg)
    S = ctx.shape[0]
    for l, d in enumerate(stack):
        x = torch.cat([ctx, h])[None]
        pos = torch.arange(x.shape[1])
        pos[S:] += shift
        mask = None
        if windows and windows[l]:
            r, c = pos[:, None], pos[None, :]
            ok = (c <= r) & (r - c < windows[l])
            mask = torch.zeros(ok.shape).masked_fill(~ok, float("-inf"))[None, None]
        pos = pos[None]
        y = d(x, attention_mask=mask, position_ids=pos, position_embeddings=rot(x, pos))
        y = y[0] if isinstance(y, tuple) else y
        h = y[0, S:]
    return h


@pytest.mark.parametrize("with_ctx,window", [(False, 0), (True, 0), (True, 4)])
def test_dflash_equals_qwen3_layer_stack(with_ctx, window):
    """window > 0: layer 0 is a sliding layer (dflash_model.py:103-109, :128-132), layer 1 full."""
    from mlx_dspark.qwen3 import TargetArgs
    g = torch.Generator().manual_seed(10 + with_ctx + window)
    a = TargetArgs(model_type="qwen3", hidden_size=256, num_hidden_layers=2, intermediate_size=384,
                   num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=500)
    tgt = OM.OracleTarget(_target(a, g))
    H, I, nq, nkv, hd = 256, 384, 4, 2, 64
    eps = 0.0 if with_ctx else 1e-6
    layers = [_layer(g, H, I, nq, nkv, hd, unit_in=with_ctx) for _ in range(2)]
    lt = ("sliding_attention", "full_attention") if window else ()
    c = types.SimpleNamespace(num_attention_heads=nq, num_key_value_heads=nkv, head_dim=hd, rms_norm_eps=eps,
                              rope_theta=1e6, layer_types=lt, sliding_window=window or None)
    wins = [window, 0] if window else None
    drafter = types.SimpleNamespace(config=c, fc=_wobj(0.05 * torch.randn(H, 2 * H, generator=g)),
                                    hidden_norm=_unit(H) if with_ctx else _norm_w(H, g), norm=_norm_w(H, g),
                                    layers=layers)
    od = OM.OracleDFlash(drafter, tgt)
    cfg, stack = _qwen3_stack(layers, H, I, nq, nkv, hd, eps, 1e6)
    fc, hn, nw = OM.deq(drafter.fc), drafter.hidden_norm.float(), drafter.norm.float()
    ctx = torch.zeros(0, H)
    for S in ([6, 3] if with_ctx else [0, 0]):       # two rounds: stored context, then new rows
        th = torch.randn(S, 2 * H, generator=g)
        ids = torch.randint(0, a.vocab_size, (5,), generator=g)
        with torch.no_grad():
            got = od(ids, th, logits_start=1)
            ctx = torch.cat([ctx, OM.rmsnorm(th @ fc.T, hn, eps)])
            want = OM.rmsnorm(_run_qwen3_stack(cfg, stack, ctx, tgt.embed[ids], windows=wins)[1:], nw, eps) \
                @ tgt.lm_head.T
            assert OM.normalized_maxdiff(got, want) < TOL
    if with_ctx:   # planted mistakes: the block roped at the context's offset instead of after it;
        with torch.no_grad():   # a window one position longer; no window at all
            bad = [_run_qwen3_stack(cfg, stack, ctx, tgt.embed[ids], shift=-3, windows=wins)]
            if window:
                bad += [_run_qwen3_stack(cfg, stack, ctx, tgt.embed[ids], windows=[window + 1, 0]),
                        _run_qwen3_stack(cfg, stack, ctx, tgt.embed[ids])]
        for hb in bad:
            assert OM.normalized_maxdiff(got, OM.rmsnorm(hb[1:], nw, eps) @ tgt.lm_head.T) > 1e-3


def _gemma4_stack(d):
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextDecoderLayer
    c = d.config
    H, I, nq, hd = c.hidden_size, c.intermediate_size, c.num_attention_heads, c.attn_head_dim
    cfg = Gemma4TextConfig(hidden_size=H, num_hidden_layers=len(d.layers), intermediate_size=I, num_attention_heads=nq,
                           num_key_value_heads=2, head_dim=64, global_head_dim=hd, num_global_key_value_heads=1,
                           attention_k_eq_v=True, vocab_size=16, rms_norm_eps=c.rms_norm_eps,
                           layer_types=["full_attention"] * len(d.layers), hidden_activation="gelu_pytorch_tanh",
                           hidden_size_per_layer_input=0, enable_moe_block=False, num_kv_shared_layers=0,
                           rope_parameters={"full_attention": {"rope_type": "proportional", "partial_rotary_factor": 0.25,
                                                               "rope_theta": 1e6},
                                            "sliding_attention": {"rope_type": "default", "rope_theta": 1e4}})
    cfg._attn_implementation = "eager"
    out = []
    for l, L in enumerate(d.layers):
        layer = Gemma4TextDecoderLayer(cfg, l).eval()
        wq = OM.deq(L.qkv)
        res = layer.load_state_dict({
            "self_attn.q_proj.weight": wq[:nq * hd], "self_attn.k_proj.weight": wq[nq * hd:(nq + 1) * hd],
            "self_attn.o_proj.weight": OM.deq(L.o), **_mlp_sd(L, I),
            "self_attn.q_norm.weight": L.q_norm.float(), "self_attn.k_norm.weight": L.k_norm.float(),
            "input_layernorm.weight": L.in_norm.float(), "post_attention_layernorm.weight": L.attn_out_norm.float(),
            "pre_feedforward_layernorm.weight": L.post_norm.float(),
            "post_feedforward_layernorm.weight": L.ff_out_norm.float(),
            "layer_scalar": torch.tensor([d.layer_scalars[l]])}, strict=False)
        assert not res.missing_keys and not res.unexpected_keys
        out.append(layer)
    return cfg, out


def _run_gemma4_stack(cfg, stack, ctx, h):
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextRotaryEmbedding
    rot = Gemma4TextRotaryEmbedding(cfg)
    S = ctx.shape[0]
    for layer in stack:
        x = torch.cat([ctx, h])[None]
        pos = torch.arange(x.shape[1])[None]
        y = layer(x, shared_kv_states={}, position_embeddings=rot(x, pos, "full_attention"), attention_mask=None,
                  position_ids=pos)
        h = y[0, S:]
    return h


@pytest.mark.parametrize("family", ["qwen3", "gemma4"])
@pytest.mark.parametrize("with_ctx", [False, True])
def test_dspark_equals_layer_stack(family, with_ctx):
    if family == "gemma4":
        pytest.importorskip("transformers.models.gemma4.modeling_gemma4")
    g = torch.Generator().manual_seed(20 + with_ctx + 2 * (family == "gemma4"))
    H, I, V = 256, 384, 500
    eps = 0.0 if with_ctx else 1e-6
    d = _dspark(g, family, H, I, V, eps, with_ctx)
    od = OM.OracleDSpark(d)
    if family == "gemma4":
        cfg, stack = _gemma4_stack(d)
        run = lambda ctx, h: _run_gemma4_stack(cfg, stack, ctx, h)
    else:
        cfg, stack = _qwen3_stack(d.layers, H, I, 4, 2, 64, eps, 1e6)
        run = lambda ctx, h: _run_qwen3_stack(cfg, stack, ctx, h)
    fc, hn, nw = OM.deq(d.fc), d.hidden_norm.float(), d.norm.float()
    scale = H ** 0.5 if family == "gemma4" else 1.0
    ctx = torch.zeros(0, H)
    for S in ([5, 3] if with_ctx else [0]):
        th = torch.randn(S, 2 * H, generator=g)
        ids = torch.randint(0, V, (6,), generator=g)
        with torch.no_grad():
            if S:
                od.update_context(th)
            got = od.block_hidden(ids)
            ctx = torch.cat([ctx, OM.rmsnorm(th @ fc.T, hn, eps)])
            want = OM.rmsnorm(run(ctx, od.embed[ids] * scale), nw, eps)
        assert float((got - want).abs().max() / want.abs().max()) < TOL
    # planted mistake on the reference side: the final norm's weight left out
    with torch.no_grad():
        bad = OM.rmsnorm(run(ctx, od.embed[ids] * scale), torch.ones(H), eps)
    assert float((got - bad).abs().max()) > 1e-2
