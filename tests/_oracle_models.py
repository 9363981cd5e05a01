"""Small random models in the layout the oracle classes read (MLX-style affine codes from
oracle/w8.py's quantizer, bf16 norm gains), built on the CPU for oracle-only tests."""

import types

import numpy as np
import torch

from oracle import w8 as W8


def _wobj(w):
    q, s, b = W8.quantize(w.numpy())
    t = lambda x: torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16)
    return types.SimpleNamespace(mlx=(torch.from_numpy(q), t(s), t(b)))


def _table(w):
    o = _wobj(w)
    return types.SimpleNamespace(q=o.mlx[0], s=o.mlx[1], b=o.mlx[2], mlx=o.mlx)


def _norm_w(n, g):
    return (1.0 + 0.3 * torch.randn(n, generator=g)).to(torch.bfloat16)


def _unit(n):
    return torch.ones(n, dtype=torch.bfloat16)


def _layer(g, H, I, nq, nkv, hd, *, sandwich=False, unit_in=False, k_eq_v=False):
    if k_eq_v:
        wk = 0.05 * torch.randn(nkv * hd, H, generator=g)
        qkv = _wobj(torch.cat([0.05 * torch.randn(nq * hd, H, generator=g), wk, wk]))
    else:
        qkv = _wobj(0.05 * torch.randn((nq + 2 * nkv) * hd, H, generator=g))
    return types.SimpleNamespace(
        qkv=qkv, o=_wobj(0.05 * torch.randn(H, nq * hd, generator=g)),
        gate_up=_wobj(0.05 * torch.randn(2 * I, H, generator=g)), down=_wobj(0.05 * torch.randn(H, I, generator=g)),
        in_norm=_unit(H) if unit_in else _norm_w(H, g), post_norm=_norm_w(H, g), q_norm=_norm_w(hd, g),
        k_norm=_norm_w(hd, g), attn_out_norm=_norm_w(H, g) if sandwich else None,
        ff_out_norm=_norm_w(H, g) if sandwich else None)


def _target(a, g):
    from mlx_dspark.qwen3 import TargetArgs  # noqa: F401  (the host-side config type)
    H, I = a.hidden_size, a.intermediate_size
    layers = [_layer(g, H, I, a.num_attention_heads, a.num_key_value_heads, a.head_dim, sandwich=a.sandwich_norms)
              for _ in range(a.num_hidden_layers)]
    emb = _table(0.5 * torch.randn(a.vocab_size, H, generator=g))
    head = types.SimpleNamespace(mlx=emb.mlx) if a.tie_word_embeddings else _wobj(
        0.05 * torch.randn(a.vocab_size, H, generator=g))
    return types.SimpleNamespace(args=a, layers=layers, embed=emb, lm_head=head, norm=_norm_w(H, g))


def _dspark(g, family, H, I, V, eps, unit):
    from mlx_dspark.config import DSparkConfig
    gemma = family == "gemma4"
    if gemma:
        c = DSparkConfig(family="gemma4", hidden_size=H, vocab_size=V, num_hidden_layers=2, intermediate_size=I,
                         rms_norm_eps=eps, num_attention_heads=4, num_key_value_heads=2, num_global_key_value_heads=1,
                         head_dim=64, global_head_dim=512, attention_k_eq_v=True, rope_theta=1e6,
                         partial_rotary_factor=0.25, rope_type="proportional", final_logit_softcapping=30.0,
                         use_v_norm=True)
    else:
        c = DSparkConfig(family="qwen3", hidden_size=H, vocab_size=V, num_hidden_layers=2, intermediate_size=I,
                         rms_norm_eps=eps, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                         attention_k_eq_v=False, rope_theta=1e6, rope_type="default", final_logit_softcapping=None,
                         use_v_norm=False, norm_style="qwen", mlp_activation="silu")
    nq, nkv, hd = c.num_attention_heads, c.n_kv_heads, c.attn_head_dim
    layers = [_layer(g, H, I, nq, nkv, hd, sandwich=gemma, unit_in=unit, k_eq_v=gemma) for _ in range(2)]
    return types.SimpleNamespace(
        config=c, layer_scalars=[0.75, 1.25] if gemma else None,
        embed_tokens=_table(0.5 * torch.randn(V, H, generator=g)), fc=_wobj(0.05 * torch.randn(H, 2 * H, generator=g)),
        hidden_norm=_unit(H) if unit else _norm_w(H, g), norm=_norm_w(H, g),
        lm_head=_wobj(0.05 * torch.randn(V, H, generator=g)), layers=layers, markov_head=None, confidence_head=None)
