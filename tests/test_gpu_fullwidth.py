"""GPU parity at the workloads' real widths, against the reference-order oracle (float32
softmax), bounded by the stated 2e-2 logits bound or by the measured noise floor where that is larger
(tests/_parity.py): the oracle against the same oracle with float64 sums, two valid evaluations
of one rounding-point graph, measured here on each case's own model and inputs.

Targets (two decoder layers each, the full vocabulary head, random norm gains):
  - Qwen3-8B shape (hidden 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU 12288) over a
    4096-token 8-bit KV context with verify blocks of 16, 47 and 64 rows;
  - Qwen3-0.6B shape (hidden 1024, 16 / 8 heads, tied head) over a 768-token bf16 context, 9 rows;
  - Gemma-style 12B shape (hidden 3840, 16 / 8 heads, head_dim 256, GeGLU 15360, 262144-row tied
    head with soft-cap 30, sandwich norms): a sliding-window (1024) layer and a global layer
    over an 8192-token bf16 context, 9 rows.
At full depth: the whole 36-layer Qwen3-8B shape, 16 rows over a 1024-token 8-bit KV context, and
the whole 48-layer Gemma-style shape, 9 rows over a 2048-token bf16 context; and the Q8 pair end to
end (36-layer target, 2-layer DFlash drafter) and the G12 pair (48-layer target, gemma4 DSpark
drafter), and the CB engine (SpecSlots, three ragged rows over the 36-layer target), their greedy
streams teacher-forced under the oracle.
The context is written straight into the paged cache (random keys and values, 8-bit quantized
with the engine's rule where the cache is 8-bit) and the oracle attends to the same values, so
the oracle only runs the verify rows.
Drafters:
  - DFlash at the Qwen3-8B width with 4-bit linears (2 layers, block 16, 5 taps) bound to the
    Qwen3-8B-width target's embedding and head, over 1024 context rows;
  - DSpark at the Qwen3-0.6B width with 4-bit linears (1 layer, taps of 3 layers, k = 8) over
    512 context rows, the block logits of 8 rows.
Context rows of the drafters are random target hidden states (rms ~2, bf16)."""

import numpy as np
import pytest
import torch

from _parity import check_greedy_stream, check_logits
from oracle import model as OM
from oracle import w8 as W8

pytestmark = pytest.mark.gpu


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


def _oracle_twice(run):
    """run(exact) -> oracle output; returns (float32 output, floor) with the floor the distance
    of the float32 evaluation from the float64-sums one."""
    want = run(False)
    exact = run(True)
    w0 = want[0] if isinstance(want, tuple) else want
    e0 = exact[0] if isinstance(exact, tuple) else exact
    return want, OM.logit_diff(w0, e0)


def _target(shape, layers=2, seed=11, **over):
    from mlx_dspark import synthetic
    args = synthetic.target_args(shape)
    args.num_hidden_layers = layers
    for k, v in over.items():
        setattr(args, k, v)
    model = synthetic.build_target(args, seed=seed, keep_mlx=True)
    synthetic.randomize_norms(model, seed=seed + 1)
    return model


CASES = [("qwen3-8b", 4096, 16, 8), ("qwen3-0.6b", 768, 9, None), ("qwen3-8b", 4096, 47, 8),
         ("qwen3-8b", 4096, 64, 8), ("gemma-12b", 8192, 9, None)]


@pytest.mark.parametrize("shape,ctx,W,kv_bits", CASES)
def test_verify_logits_full_width(dev, shape, ctx, W, kv_bits):
    print(f"full-width verify {shape} ctx={ctx} W={W} kv_bits={kv_bits}", flush=True)
    over = {}
    if shape == "gemma-12b":   # one sliding-window layer and one global layer
        over["layer_types"] = ("sliding_attention", "full_attention")
    model = _target(shape, **over)
    a = model.args
    nkv, hd = a.num_key_value_heads, a.head_dim
    cache = model.make_cache(max_ctx=ctx + 64, kv_bits=kv_bits)
    g = torch.Generator().manual_seed(13)
    ref = OM.OracleTarget(model, kv_bits=kv_bits)
    held = []
    for l in range(a.num_hidden_layers):
        K = 0.4 * torch.randn(ctx, nkv, hd, generator=g)
        V = torch.randn(ctx, nkv, hd, generator=g)
        held.append(_fill_context(cache, l, K, V))
    cache.set_lengths([ctx])
    block = torch.randint(0, a.vocab_size, (W,), generator=g)
    ids = block.to(dev, torch.int32).view(1, W)
    logits, fused = model.forward(ids, cache, [0], advance=False)
    torch.cuda.synchronize()
    got = logits[0].float().cpu()

    def run(exact):
        ref.K = [k for k, _ in held]
        ref.V = [v for _, v in held]
        ref.offset = ctx
        with OM.exact_sums(exact):
            return ref.forward(block, tap=(0,))

    (rl, rf), floor = _oracle_twice(run)
    check_logits(got, rl, f"{shape} verify logits", floor=floor)
    if a.final_logit_softcapping:
        assert float(got.abs().max()) <= a.final_logit_softcapping
    tap = float((fused[0].float().cpu() - rf).abs().max() / rf.abs().max())
    print(f"  tap: max-abs relative {tap:.4f}", flush=True)
    assert tap < 2e-2


def test_dflash_drafter_full_width(dev):
    """DFlash (src/mlx_dspark/dflash_model.py:197-208) at the Qwen3-8B width, 4-bit linears,
    bound to a Qwen3-8B-width target's embedding and W8 head; two rounds (1024, then 5 more
    context rows)."""
    from mlx_dspark import synthetic
    print("full-width DFlash drafter: qwen3-8b width, 4-bit, block 16, 5 taps, 1024 context rows", flush=True)
    model = _target("qwen3-8b")
    full = synthetic.target_args("qwen3-8b")       # 36-layer tap ids; the rows below are random
    d, cfg = synthetic.build_dflash(full, seed=9, keep_mlx=True, num_hidden_layers=2, block_size=16, n_taps=5)
    synthetic.randomize_norms(d, seed=10)
    d.bind(model)
    H, V = full.hidden_size, full.vocab_size
    g = torch.Generator().manual_seed(5)
    ctx = (2.0 * torch.randn(1024, 5 * H, generator=g)).to(torch.bfloat16)
    more = (2.0 * torch.randn(5, 5 * H, generator=g)).to(torch.bfloat16)
    block = [int(torch.randint(0, V, (1,), generator=g))] + [cfg.mask_token_id] * (cfg.block_size - 1)
    dcache = d.make_cache(max_ctx=2048)
    got1 = d(block, ctx.to(dev), dcache, logits_start=1)[0].float().cpu()
    got2 = d(block, more.to(dev), dcache, logits_start=1)[0].float().cpu()
    torch.cuda.synchronize()
    ref_t = OM.OracleTarget(model)

    def run(exact):
        od = OM.OracleDFlash(d, ref_t)
        with OM.exact_sums(exact):
            return od(block, ctx.float(), logits_start=1), od(block, more.float(), logits_start=1)

    w1, w2 = run(False)
    e1, e2 = run(True)
    check_logits(got1, w1, "dflash round 1 (1024 context rows)", floor=OM.logit_diff(w1, e1))
    check_logits(got2, w2, "dflash round 2 (5 more rows)", floor=OM.logit_diff(w2, e2))


def test_dspark_drafter_full_width(dev):
    """DSpark (src/mlx_dspark/model.py:244-309) at the Qwen3-0.6B width, 4-bit linears and
    tables: context ingest of 512 rows, the 8-row block's logits."""
    from mlx_dspark import synthetic
    print("full-width DSpark drafter: qwen3-0.6b width, 4-bit, k = 8, 512 context rows", flush=True)
    full = synthetic.target_args("qwen3-0.6b")
    d, cfg = synthetic.build_dspark(full, seed=7, keep_mlx=True, num_hidden_layers=1, block_size=8,
                                    taps=[1, 14, 27])
    synthetic.randomize_norms(d, seed=8)
    H, V = full.hidden_size, full.vocab_size
    g = torch.Generator().manual_seed(6)
    ctx = (2.0 * torch.randn(512, 3 * H, generator=g)).to(torch.bfloat16)
    dcache = d.make_ctx_cache(max_ctx=1024)
    d.update_context(ctx.to(dev), 0, dcache)
    block = torch.tensor([[int(torch.randint(0, V, (1,), generator=g))] + [cfg.mask_token_id] * (cfg.block_size - 1)],
                         dtype=torch.int32, device=dev)
    got = d.block_logits(block, dcache, cfg.block_size)[0].float().cpu()
    torch.cuda.synchronize()

    def run(exact):
        od = OM.OracleDSpark(d)
        with OM.exact_sums(exact):
            od.update_context(ctx.float())
            return od.base_logits(block.cpu()[0], cfg.block_size)

    want, floor = _oracle_twice(run)
    check_logits(got, want, "dspark block logits (512 context rows)", floor=floor)


def test_verify_logits_full_depth_qwen3_8b(dev):
    """The whole 36-layer Qwen3-8B-shaped target (random norm gains), a 16-row verify over a
    1024-token 8-bit KV context in every layer, against the oracle at full depth: the rounding
    differences of 36 layers compound in the residual stream, and the floor measured on the
    same model and inputs grows with them, so the bound is the same rule as at two layers."""
    print("full-depth verify qwen3-8b: 36 layers, ctx=1024, W=16, 8-bit KV", flush=True)
    model = _target("qwen3-8b", layers=36, seed=21)
    a = model.args
    nkv, hd, ctx, W = a.num_key_value_heads, a.head_dim, 1024, 16
    cache = model.make_cache(max_ctx=ctx + 64, kv_bits=8)
    g = torch.Generator().manual_seed(23)
    held = []
    for l in range(a.num_hidden_layers):
        K = 0.4 * torch.randn(ctx, nkv, hd, generator=g)
        V = torch.randn(ctx, nkv, hd, generator=g)
        held.append(_fill_context(cache, l, K, V))
    cache.set_lengths([ctx])
    block = torch.randint(0, a.vocab_size, (W,), generator=g)
    ids = block.to(dev, torch.int32).view(1, W)
    logits, _ = model.forward(ids, cache, None, advance=False)
    torch.cuda.synchronize()
    got = logits[0].float().cpu()
    ref = OM.OracleTarget(model, kv_bits=8)

    def run(exact):
        ref.K = [k for k, _ in held]
        ref.V = [v for _, v in held]
        ref.offset = ctx
        with OM.exact_sums(exact):
            return ref.forward(block)[0]

    rl, floor = _oracle_twice(run)
    check_logits(got, rl, "qwen3-8b 36-layer verify logits", floor=floor)
    # the greedy picks the verify decides: the GPU's argmax is the oracle's, or within the
    # bound of the oracle's best normalised logit
    rn = rl / rl.pow(2).mean(-1, keepdim=True).sqrt()
    pick = got.argmax(-1)
    gap = rn.max(-1).values - rn.gather(1, pick[:, None])[:, 0]
    print(f"  greedy picks: {int((gap == 0).sum())}/{W} are the oracle's argmax, largest gap "
          f"{float(gap.max()):.4f}", flush=True)
    assert float(gap.max()) <= max(2e-2, 1.5 * floor[0])


def test_verify_logits_full_depth_gemma_12b(dev):
    """The whole 48-layer Gemma-style 12B target (40 sliding-window layers of 1024 keys, 8 global
    ones, sandwich norms, soft-capped 262144-row head; random norm gains), a 9-row verify over a
    2048-token bf16 context in every layer, against the oracle at full depth with the same
    floor rule."""
    print("full-depth verify gemma-12b: 48 layers, ctx=2048, W=9, bf16 KV", flush=True)
    model = _target("gemma-12b", layers=48, seed=31)
    a = model.args
    nkv, hd, ctx, W = a.num_key_value_heads, a.head_dim, 2048, 9
    assert sum(a.is_sliding(l) for l in range(a.num_hidden_layers)) == 40
    cache = model.make_cache(max_ctx=ctx + 64, kv_bits=None)
    g = torch.Generator().manual_seed(33)
    held = []
    for l in range(a.num_hidden_layers):
        K = 0.4 * torch.randn(ctx, nkv, hd, generator=g)
        V = torch.randn(ctx, nkv, hd, generator=g)
        held.append(_fill_context(cache, l, K, V))
    cache.set_lengths([ctx])
    block = torch.randint(0, a.vocab_size, (W,), generator=g)
    ids = block.to(dev, torch.int32).view(1, W)
    logits, _ = model.forward(ids, cache, None, advance=False)
    torch.cuda.synchronize()
    got = logits[0].float().cpu()
    assert float(got.abs().max()) <= a.final_logit_softcapping
    ref = OM.OracleTarget(model, kv_bits=None)

    def run(exact):
        ref.K = [k for k, _ in held]
        ref.V = [v for _, v in held]
        ref.offset = ctx
        with OM.exact_sums(exact):
            return ref.forward(block)[0]

    rl, floor = _oracle_twice(run)
    check_logits(got, rl, "gemma-12b 48-layer verify logits", floor=floor)
    rn = rl / rl.pow(2).mean(-1, keepdim=True).sqrt()
    pick = got.argmax(-1)
    gap = rn.max(-1).values - rn.gather(1, pick[:, None])[:, 0]
    print(f"  greedy picks: {int((gap == 0).sum())}/{W} are the oracle's argmax, largest gap "
          f"{float(gap.max()):.4f}", flush=True)
    assert float(gap.max()) <= max(2e-2, 1.5 * floor[0])


def test_q8_dflash_stream_full_depth(dev):
    """The Q8 pair end to end at full depth: the 36-layer Qwen3-8B-shaped W8 target with 8-bit KV
    and the 2-layer 4-bit DFlash drafter (block 16) decode 32 tokens after a 64-token prompt in
    graph-replayed rounds; the stream, teacher-forced under the oracle's 36-layer target with the
    same 8-bit cache, is the oracle's greedy decoding under the margin rule."""
    from mlx_dspark import synthetic
    from mlx_dspark.generate import dflash_generate
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    print("Q8 pair at full depth: 36-layer W8 target, 8-bit KV, 2-layer 4-bit DFlash, 32 tokens", flush=True)
    model = synthetic.build_target("qwen3-8b", seed=41, keep_mlx=True)
    tok = SyntheticTokenizer(model.args.vocab_size)
    target = Target(model, tok, kv_bits=8)
    d, _ = synthetic.build_dflash(model.args, seed=42, block_size=16, n_taps=5, bits=4)
    d.bind(model)
    prompt = np.random.default_rng(43).integers(0, model.args.vocab_size, 64).tolist()
    r = dflash_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=32, use_graph=True)
    s = r.token_ids[:32]
    assert len(s) == 32 and r.num_rounds >= 8
    check_greedy_stream(model, prompt, s, 24, kv_bits=8)


def test_g12_dspark_stream_full_depth(dev):
    """The G12 pair end to end at full depth: the 48-layer Gemma-style W8 target (40 sliding
    layers) with 8-bit KV and the 1-layer gemma4 DSpark drafter decode 24 greedy tokens (block 8,
    lookup drafts off) after a 64-token prompt; the stream, teacher-forced under the oracle's
    48-layer target with the same 8-bit cache, is the oracle's greedy decoding under the margin
    rule."""
    from mlx_dspark import synthetic
    from mlx_dspark.generate import speculative_generate
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    print("G12 pair at full depth: 48-layer W8 target, 8-bit KV, gemma4 DSpark, 24 tokens", flush=True)
    model = synthetic.build_target("gemma-12b", seed=51, keep_mlx=True)
    d, _ = synthetic.build_dspark(model.args, seed=52, num_hidden_layers=1, block_size=8, family="gemma4")
    tok = SyntheticTokenizer(model.args.vocab_size)
    target = Target(model, tok, kv_bits=8)
    prompt = np.random.default_rng(53).integers(0, model.args.vocab_size, 64).tolist()
    r = speculative_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=24, max_draft_tokens=8,
                             lookup_drafts=False)
    s = r.token_ids[:24]
    assert len(s) == 24
    check_greedy_stream(model, prompt, s, 18, kv_bits=8)


def test_cb_slots_greedy_full_depth(dev):
    """The CB engine at full depth: SpecSlots over the 36-layer Qwen3-8B-shaped W8 target with
    8-bit KV and a 1-layer DSpark drafter (8 drafts, W = 9), three rows with ragged prompts
    decoding greedily together; each row's stream, teacher-forced under the oracle's 36-layer
    target with the same 8-bit cache, is the oracle's greedy decoding under the margin rule."""
    from mlx_dspark import synthetic
    from mlx_dspark.batch_engine import SpecSlots
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    print("CB engine at full depth: 36-layer W8 target, 8-bit KV, DSpark k = 8, 3 ragged rows", flush=True)
    model = synthetic.build_target("qwen3-8b", seed=61, keep_mlx=True)
    tok = SyntheticTokenizer(model.args.vocab_size)
    target = Target(model, tok, kv_bits=8)
    d, _ = synthetic.build_dspark(model.args, seed=62, num_hidden_layers=1, block_size=8)
    rng = np.random.default_rng(63)
    prompts = [rng.integers(0, model.args.vocab_size, n).tolist() for n in (40, 72, 24)]
    slots = SpecSlots(target, tok, d, capacity=3, max_draft_tokens=8, max_ctx=256)
    for i, p in enumerate(prompts):
        slots.admit(p, max_new_tokens=16, meta=i)
    done, rounds = {}, 0
    while slots.n_active:
        for meta, r in slots.step():
            done[meta] = r
        rounds += 1
        assert rounds < 100
    for i, p in enumerate(prompts):
        s = done[i].token_ids[:16]
        assert len(s) == 16
        check_greedy_stream(model, p, s, 12, kv_bits=8)
