"""Rounding sources of the verify forward at the Qwen3-8B width, measured on the CPU.

Two decoder layers of the Qwen3-8B shape (hidden 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU
12288, a 151936-row head, tied here so one table is built), random N(0, 0.02) weights quantized
8-bit group 64, random norm gains, a 4096-token 8-bit context of random keys (0.4 N(0, 1)) and
values (N(0, 1)) and a 16-row verify block: the shapes of tests/test_gpu_fullwidth.py. The
reference-order oracle (float32 softmax; the Qwen3 layout's norms applied after the projections,
as the engine applies them) is compared in the logits tolerance's metric (max-abs and rms of the
difference of RMS-normalised logit rows) with
  - the same rounding points evaluated with float64 sums (oracle.model.exact_sums): two valid
    evaluations of one rounding-point graph, whose distance is the metric's noise floor here;
  - the oracle with one rounding choice changed at a time.

The random model amplifies small differences: its embedding rows and first attention output are
~0.02 in size against ~2.4 for the first MLP's output, so the first MLP, which normalises its
input, passes a relative change of the first layer's small terms on to the whole residual
stream, and every later bf16 rounding that such a change flips passes on a whole bf16 step.

Asserted: the floor is above 2e-2 at this width (so the full-width GPU tests bound the logits by
the measured floor); the split kernels' evaluation order with float32 probabilities and partials
(256-key splits, one max per 64 keys, the exp2 form) stays within the floor; and bf16
probabilities, bf16 split partials and the float32-revolution form of the RoPE sine each move
the logits past 2e-2 (why the attention kernels carry P as three bf16 terms, keep float32 split
partials and take the sine of the float32 angle with a full argument reduction).
"""

import time
import types

import numpy as np
import pytest
import torch

from oracle import model as OM
from _oracle_models import _norm_w, _wobj

H, I, NQ, NKV, HD, V = 4096, 12288, 32, 8, 128, 151936
CTX, W = 4096, 16


@pytest.fixture(scope="module")
def fullwidth():
    from mlx_dspark.qwen3 import TargetArgs
    t0 = time.time()
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    g = torch.Generator().manual_seed(21)
    a = TargetArgs(model_type="qwen3", hidden_size=H, num_hidden_layers=2, intermediate_size=I,
                   num_attention_heads=NQ, num_key_value_heads=NKV, head_dim=HD, vocab_size=V,
                   tie_word_embeddings=True)
    def w(n, k):
        return _wobj(0.02 * torch.randn(n, k, generator=g))
    layers = []
    for _ in range(2):
        layers.append(types.SimpleNamespace(
            qkv=w((NQ + 2 * NKV) * HD, H), o=w(H, NQ * HD), gate_up=w(2 * I, H), down=w(H, I),
            in_norm=_norm_w(H, g), post_norm=_norm_w(H, g),
            q_norm=(HD ** -0.25 * (1 + 0.3 * torch.randn(HD, generator=g))).to(torch.bfloat16),
            k_norm=(HD ** -0.25 * (1 + 0.3 * torch.randn(HD, generator=g))).to(torch.bfloat16),
            attn_out_norm=None, ff_out_norm=None))
    head = w(V, H)
    emb = types.SimpleNamespace(q=head.mlx[0], s=head.mlx[1], b=head.mlx[2], mlx=head.mlx)
    model = types.SimpleNamespace(args=a, layers=layers, embed=emb, lm_head=head, norm=_norm_w(H, g))
    ot = OM.OracleTarget(model, kv_bits=8)
    ctx = [(OM.kv_quant_roundtrip(0.4 * torch.randn(CTX, NKV, HD, generator=g)),
            OM.kv_quant_roundtrip(torch.randn(CTX, NKV, HD, generator=g))) for _ in range(2)]
    block = torch.randint(0, V, (W,), generator=g)
    print(f"full-width CPU model built in {time.time() - t0:.1f} s", flush=True)
    return ot, ctx, block


def _run(fw, *, exact=False, **knobs):
    ot, ctx, block = fw
    base = dict(p_bf16=False, norm_first=False, rope_revolutions=False, requant_new=True,
                rr=lambda x: x, attn_opts=dict(split=0, block=0, partial_bf16=False, exp2=False, terms=0))
    opts = dict(base)
    attn = dict(base["attn_opts"])
    for k, v in knobs.items():
        if k in attn or k == "p_terms":
            attn["terms" if k == "p_terms" else k] = v
        elif k == "double_round":
            opts["rr"] = OM.bf if v else (lambda x: x)
        else:
            opts[k] = v
    opts["attn_opts"] = attn
    for k, v in opts.items():
        setattr(ot, k, v)
    ot.K = [k for k, _ in ctx]
    ot.V = [v for _, v in ctx]
    ot.offset = CTX
    with OM.exact_sums(exact):
        logits, _ = ot.forward(block)
    return logits


KERNEL_ORDER = dict(split=256, block=64, exp2=True)   # the verify kernel's splits, waves and exp form


def test_rounding_sources(fullwidth):
    ref = _run(fullwidth)
    rows = {
        "float64 sums (the floor)": dict(exact=True),
        "split-kernel order, float32 P and partials": dict(KERNEL_ORDER),
        "  + float64 sums": dict(KERNEL_ORDER, exact=True),
        "bf16 P (one max per row)": dict(p_bf16=True),
        "two-term P (hi + lo, the many-query prefill kernel)": dict(KERNEL_ORDER, p_terms=2),
        "bf16 P, one max per 64 keys, bf16 256-key partials": dict(KERNEL_ORDER, p_bf16=True, partial_bf16=True),
        "bf16 256-key split partials (float32 P)": dict(KERNEL_ORDER, partial_bf16=True),
        "RoPE sine of float32 revolutions": dict(rope_revolutions=True),
        "exp2 form (kernel) instead of exp": dict(exp2=True),
        "new K/V rows kept bf16 (no 8-bit re-quantisation)": dict(requant_new=False),
        "norms before the projections (unfused graph order)": dict(norm_first=True),
        "projection outputs rounded before the residual add": dict(double_round=True),
    }
    res = {}
    print("\nsource (alone, against the reference order)                 max-abs      rms", flush=True)
    for name, knobs in rows.items():
        got = _run(fullwidth, **knobs)
        res[name] = OM.logit_diff(got, ref)
        print(f"{name:60s} {res[name][0]:8.4f} {res[name][1]:9.5f}", flush=True)
    floor = res["float64 sums (the floor)"][0]
    assert floor > 2e-2, "the floor is below the nominal tolerance at this width"
    assert res["split-kernel order, float32 P and partials"][0] <= floor
    for src in ("bf16 P (one max per row)", "bf16 256-key split partials (float32 P)", "RoPE sine of float32 revolutions"):
        assert res[src][0] > 2e-2, src
