"""GPU parity of the verify forward at the workloads' real widths: two decoder layers of the
Qwen3-8B shape (hidden 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU 12288) over a 4096-token
8-bit KV context with a 16-row verify block, and two layers of the Qwen3-0.6B shape (hidden
1024, 16 / 8 heads, tied head) over a 768-token bf16 context with a 9-row block, each with the
full 151936-row vocabulary head and random norm gains. The context is written straight into the
paged cache (random keys and values, 8-bit quantized with the engine's rule where the cache is
8-bit) and the oracle attends to the same dequantized values, so the oracle only runs the
verify rows."""

import numpy as np
import pytest
import torch

from _parity import check_logits
from oracle import model as OM
from oracle import w8 as W8

pytestmark = pytest.mark.gpu

# Logits are held to the metric's bf16 noise floor, measured in the test (tests/_parity.py); the
# rms of the difference also stays below an absolute 1.5e-2.
RMS_ABS = 1.5e-2


def _fill_context(cache, l, K, V):
    """Write K, V [L, nkv, hd] (float) as the cache's first L tokens of layer l; returns the
    values the cache holds (bf16, or the 8-bit round trip)."""
    L, nkv, hd = K.shape
    page = cache.page
    held = []
    for src, pool, sb in ((K, cache.k[l], cache.k_sb[l]), (V, cache.v[l], cache.v_sb[l])):
        x = src.reshape(L * nkv, hd).numpy().astype(np.float32)
        if sb is None:
            xb = torch.from_numpy(x).to(torch.bfloat16).view(L, nkv, hd)
            dst = pool.view(-1, nkv, page, hd)
            for t0 in range(0, L, page):
                n = min(page, L - t0)
                dst[t0 // page, :, :n] = xb[t0:t0 + n].transpose(0, 1).to(pool.device)
            held.append(xb.float())
        else:
            q, s16, b16 = W8.quantize(x)
            held.append(OM.bf(torch.from_numpy(W8.dequantize(q, s16, b16).astype(np.float32))).view(L, nkv, hd))
            qv = torch.from_numpy(q).view(L, nkv, hd)
            sbv = torch.from_numpy((s16.astype(np.uint32) | (b16.astype(np.uint32) << 16)).view(np.int32)).view(
                L, nkv, hd // 64)
            for t0 in range(0, L, page):
                n = min(page, L - t0)
                pool[t0 // page, :, :n] = qv[t0:t0 + n].transpose(0, 1).to(pool.device)
                sb[t0 // page, :, :n] = sbv[t0:t0 + n].transpose(0, 1).to(sb.device)
    return held


@pytest.mark.parametrize("shape,ctx,W,kv_bits", [("qwen3-8b", 4096, 16, 8), ("qwen3-0.6b", 768, 9, None),
                                                  ("qwen3-8b", 4096, 47, 8), ("qwen3-8b", 4096, 64, 8)])
def test_verify_logits_full_width(dev, shape, ctx, W, kv_bits):
    from mlx_dspark import synthetic
    print(f"full-width verify {shape} ctx={ctx} W={W} kv_bits={kv_bits}", flush=True)
    args = synthetic.target_args(shape)
    args.num_hidden_layers = 2
    model = synthetic.build_target(args, seed=11, keep_mlx=True)
    synthetic.randomize_norms(model, seed=12)
    a = model.args
    nkv, hd = a.num_key_value_heads, a.head_dim
    cache = model.make_cache(max_ctx=ctx + 64, kv_bits=kv_bits)
    g = torch.Generator().manual_seed(13)
    refs = {"fp32 softmax": OM.OracleTarget(model, kv_bits=kv_bits),
            "bf16 probabilities": OM.OracleTarget(model, kv_bits=kv_bits, p_bf16=True)}
    for l in range(a.num_hidden_layers):
        K = 0.4 * torch.randn(ctx, nkv, hd, generator=g)
        V = torch.randn(ctx, nkv, hd, generator=g)
        Kh, Vh = _fill_context(cache, l, K, V)
        for r in refs.values():
            r.K[l], r.V[l] = Kh, Vh
    for r in refs.values():
        r.offset = ctx
    cache.set_lengths([ctx])
    block = torch.randint(0, a.vocab_size, (W,), generator=g)
    ids = block.to(dev, torch.int32).view(1, W)
    logits, fused = model.forward(ids, cache, [0], advance=False)
    torch.cuda.synchronize()
    got = logits[0].float().cpu()
    outs = {name: r.forward(block, tap=(0,)) for name, r in refs.items()}
    floor_max, floor_rms = OM.logit_diff(outs["fp32 softmax"][0], outs["bf16 probabilities"][0])
    print(f"  oracle vs oracle (softmax rounding only): normalised max-abs {floor_max:.4f} rms {floor_rms:.5f}",
          flush=True)
    for name, (rl, rf) in outs.items():
        mx, rms = OM.logit_diff(got, rl)
        tap = float((fused[0].float().cpu() - rf).abs().max() / rf.abs().max())
        print(f"  GPU vs oracle with {name}: normalised max-abs {mx:.4f} rms {rms:.5f}; tap rel {tap:.4f}", flush=True)
    check_logits(got, outs["bf16 probabilities"][0], outs["fp32 softmax"][0], f"{shape} verify logits")
    assert OM.logit_diff(got, outs["bf16 probabilities"][0])[1] < RMS_ABS
    tap = float((fused[0].float().cpu() - outs["bf16 probabilities"][1]).abs().max()
                / outs["bf16 probabilities"][1].abs().max())
    assert tap < 2e-2
