#!/usr/bin/env python
"""Benchmark of the speculative-decoding verify engine on one MI355X.

Workload (the config the headline metric is quoted on): a Qwen3-8B-shaped random-init W8
target (36 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU 12288, vocab 151936)
with a 2-layer DFlash block-diffusion drafter (4-bit linear layers, as the reference quantizes
drafters) conditioned on 5 evenly spaced target layers;
batch 1, a seeded 4096-token context, the full 16-position block verified every round
(anchor + 15 drafts), 8-bit affine KV cache (group 64), greedy acceptance.

A "step" is one speculative round: draft the block, verify it in one target forward, accept,
roll the KV back and grow the drafter context. Rounds from the second on are one HIP-graph
replay each. Printed (one JSON line):
  value        accepted tokens per second over the timed rounds (with random weights the
               drafter almost never matches, so ~1 token per round: accept length is reported)
  verify_us    one verify forward (16 rows, 4096 context), graph-replayed, HIP events
  verify_roofline_frac  algorithmic bytes of that forward / verify_us / 8 TB/s
  roofline     the dominant kernel, the W8 GEMM at the gate_up shape (24576 x 4096, SwiGLU
               epilogue): algorithmic bytes per launch over its in-graph average launch time
               (36 launches, one per layer's weights, HIP events on the launch stream)
  cpu_baseline the CPU oracle (torch, float32) on a bounded sample: one decoder layer and the
               vocabulary head of the verify step, scaled to a whole round
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "mlx-dspark_amd"))
sys.path.insert(0, str(REPO))

PEAK_HBM_GBS = 8000.0
# HBM bytes per gate_up launch from the FETCH_SIZE / WRITE_SIZE counter runs of
# `bench.py --roofline-only` (profiles/w8_gemm_gate_up_24576x4096_m16_counters.md): fetches
# 52778.54 KiB x 2.000 + writes 384 KiB x 1.000, the scales read on a 256 MiB copy
TRAFFIC_GATE_UP = 108483666


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_bytes_per_token(args, kv_bits) -> int:
    per_head = args.head_dim * 2 if kv_bits is None else args.head_dim + 4 * (args.head_dim // 64)
    return 2 * per_head * args.num_key_value_heads * args.num_hidden_layers


def gemm_roofline(model, M: int, reps: int = 10):
    """In-graph average launch duration of the W8 GEMM at every verify-step shape, with the
    epilogue the forward uses (split-K partials for qkv / o / down, fused SwiGLU for gate_up,
    f32 logits for the head). One CUDA graph per shape holds one launch per layer, each on
    that layer's weights (so every launch streams its weights from HBM), replayed `reps` times
    between two HIP events recorded on the launch stream; the average includes the ~1.5 us
    dispatch gap between back-to-back graph kernels, which a kernel trace does not count."""
    import torch
    from mlx_dspark import ops

    dev = model.device
    P, SW = ops.DSK_EPI_PARTIAL, ops.DSK_EPI_SWIGLU
    shapes = {"qkv": ([L.qkv for L in model.layers], P), "o": ([L.o for L in model.layers], P),
              "gate_up": ([L.gate_up for L in model.layers], SW), "down": ([L.down for L in model.layers], P),
              "lm_head": ([model.lm_head], ops.DSK_EPI_STORE)}
    res = {}
    stream = torch.cuda.current_stream()
    for name, (ws, epi) in shapes.items():
        K = ws[0].K
        x = ops.pack(torch.randn(M, K, device=dev).to(torch.bfloat16))
        out = None
        if epi == ops.DSK_EPI_STORE:
            out = torch.empty(M, ws[0].N, device=dev, dtype=torch.float32)
        y = ops.w8_gemm(x, ws[0], epi=epi, out=out)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for w in ws:
                ops.w8_gemm(x, w, epi=epi, out=y)
        for _ in range(2):
            g.replay()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s_ev.record(stream)
        for _ in range(reps):
            g.replay()
        e_ev.record(stream)
        torch.cuda.synchronize()
        us = s_ev.elapsed_time(e_ev) * 1e3 / (reps * len(ws))
        # algorithmic bytes: weights (q + scale/bias) + activation in + output out
        out_b = {P: 4 * ops.gemm_splits(M, ws[0].N, K), SW: 1, ops.DSK_EPI_STORE: 4}[epi] * M * ws[0].N
        by = ws[0].N * K * 1.0625 + M * K * 2 + out_b
        res[name] = {"us": round(us, 2), "bytes": int(by), "GBs": round(by / us / 1e3, 1), "launches": len(ws)}
        del g
    return res


ACC_SHAPE = (4, 16, 151936)   # batch, drafts per row, vocabulary


def acc_inputs(seed: int = 2024):
    """The standalone acceptance workload: draft logits N(0, 3^2) [4, 16, 151936], target logits
    = draft + N(0, 1) [4, 17, 151936] (the 17th row draws the bonus), drafts = the draft argmax."""
    import torch
    B, L, V = ACC_SHAPE
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L + 1, V, generator=g) * 3.0
    p = q + torch.randn(B, L + 1, V, generator=g)
    q = q[:, :L].contiguous()
    draft = q.argmax(dim=2).to(torch.int32)
    return p, q, draft


def acc_timing(reps: int = 50):
    """Speculative-sampling acceptance on [4, 17, 151936] fp32 (T = 1, top-p 0.95, top-k 0,
    Philox uniforms), inputs resident in HBM: one captured graph of the whole acceptance
    (its kernel chain, rollback included) replayed `reps` times between HIP events on the
    launch stream. Algorithmic bytes: one pass over the target and draft logits."""
    import torch
    from mlx_dspark import ops
    p, q, draft = (t.cuda() for t in acc_inputs())
    B = p.shape[0]
    sl = torch.zeros(B, dtype=torch.int32, device="cuda")
    n = torch.empty(B, dtype=torch.int32, device="cuda")
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    word = torch.zeros(1, dtype=torch.int32, device="cuda")
    run = lambda: ops.accept_sample(p, q, draft, 1.0, 0.95, 0, seed=7, offset_dev=word, seq_lens=sl, n_out=n,
                                    token_out=tok)
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    for _ in range(3):
        g.replay()
    stream = torch.cuda.current_stream()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s_ev.record(stream)
    for _ in range(reps):
        g.replay()
    e_ev.record(stream)
    torch.cuda.synchronize()
    us = s_ev.elapsed_time(e_ev) * 1e3 / reps
    nbytes = (p.numel() + q.numel()) * 4
    return {"us": round(us, 2), "bytes": int(nbytes), "GBs": round(nbytes / us / 1e3, 1),
            "roofline_frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
            "config": "B=4, 16 drafts + bonus, V=151936 fp32, T=1, top_p=0.95, top_k=0"}


def copy_calibration(nbytes: int = 256 << 20) -> None:
    """A plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def cpu_baseline(tgt_args, dev_model_seed: int, ctx: int, W: int, mean_accept: float, budget_s: float = 12.0):
    """The oracle (torch on the host CPU, float32 with bf16 rounding points) on one decoder
    layer + the vocabulary head of one verify step at the same shapes; a round is scaled as
    (target layers + drafter layers) * t_layer + 2 * t_head (target verify head + drafter head)."""
    import types

    import numpy as np
    import torch

    from mlx_dspark import synthetic
    from oracle import model as OM

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    a = tgt_args
    H, I = a.hidden_size, a.intermediate_size
    nq, nkv, hd = a.num_attention_heads, a.num_key_value_heads, a.head_dim

    def mlx(N, K, name):
        w = synthetic.randn((N, K), dev_model_seed, name, "cuda")
        from mlx_dspark.ops import W8Weight
        q, s, b = W8Weight.quantize_mlx(w)
        o = types.SimpleNamespace(mlx=(q.cpu(), s.cpu(), b.cpu()))
        return o

    ones = lambda n: torch.ones(n, dtype=torch.bfloat16)
    qk = lambda: torch.full((hd,), hd ** -0.25).to(torch.bfloat16)
    layer = types.SimpleNamespace(qkv=mlx(a.n_qkv, H, "layers.0.qkv"), o=mlx(H, nq * hd, "layers.0.o"),
                                  gate_up=mlx(2 * I, H, "layers.0.gate_up"), down=mlx(H, I, "layers.0.down"),
                                  in_norm=ones(H), post_norm=ones(H), q_norm=qk(), k_norm=qk())
    emb = mlx(a.vocab_size, H, "embed_tokens").mlx
    head = mlx(a.vocab_size, H, "lm_head")
    m = types.SimpleNamespace(args=a, layers=[layer], embed=types.SimpleNamespace(q=emb[0], s=emb[1], b=emb[2]),
                              lm_head=head, norm=ones(H))
    ref = OM.OracleTarget(m)
    g = torch.Generator().manual_seed(0)
    t_all, t_head = [], []
    ids = torch.randint(0, a.vocab_size, (W,), generator=g)
    t_start = time.perf_counter()
    while len(t_all) < 3 or time.perf_counter() - t_start < budget_s:
        ref.K = [OM.bf(torch.randn(ctx, nkv, hd, generator=g))]
        ref.V = [OM.bf(torch.randn(ctx, nkv, hd, generator=g))]
        ref.offset = ctx
        t0 = time.perf_counter()
        ref.forward(ids)
        t_all.append(time.perf_counter() - t0)
        x = torch.randn(W, H, generator=g)
        t0 = time.perf_counter()
        _ = OM.bf(x) @ ref.lm_head.T
        t_head.append(time.perf_counter() - t0)
    ta, th = statistics.median(t_all), statistics.median(t_head)
    t_layer = max(ta - th, 1e-6)
    n_layers_round = a.num_hidden_layers + 2
    t_round = n_layers_round * t_layer + 2 * th
    sample_s = sum(t_all) + sum(t_head)
    return {"value": round(mean_accept / t_round, 4), "unit": "accepted tok/s", "cores": ncores, "kind": "port",
            "sample": (f"oracle (torch fp32, bf16 rounding points) timed on 1 of {a.num_hidden_layers} decoder "
                       f"layers + the {a.vocab_size}-row head for one {W}-row verify at {ctx} context "
                       f"(median of {len(t_all)}, {sample_s:.1f} s of CPU work); round = "
                       f"{n_layers_round} layers x {t_layer * 1e3:.1f} ms + 2 heads x {th * 1e3:.1f} ms = "
                       f"{t_round * 1e3:.0f} ms, x mean accept length {mean_accept:.2f}")}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--block", type=int, default=16)
    ap.add_argument("--kv-bits", type=int, default=8, choices=[0, 8])
    ap.add_argument("--target", default="qwen3-8b")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--verify-reps", type=int, default=50)
    ap.add_argument("--roofline-only", action="store_true",
                    help="build the target, time the W8 GEMM shapes and a 256 MiB copy only (counter runs)")
    ap.add_argument("--acc-only", action="store_true",
                    help="time the standalone acceptance workload [4, 17, 151936] only")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this engine has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from mlx_dspark import ops, synthetic
    from mlx_dspark.generate import _DFlashRound, _pick
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer

    kv_bits = args.kv_bits or None
    torch.cuda.init()
    if args.acc_only:
        print(json.dumps({"acc": acc_timing()}), flush=True)
        return 0
    t_build = time.time()
    model = synthetic.build_target(args.target, seed=0)
    drafter, dcfg = synthetic.build_dflash(model.args, seed=1, block_size=args.block, n_taps=5, bits=4)
    drafter.bind(model)
    log(f"built {args.target} W8 target ({model.weight_bytes / 1e9:.2f} GB) + DFlash drafter in "
        f"{time.time() - t_build:.1f} s")
    if args.roofline_only:
        shapes = gemm_roofline(model, args.block)
        copy_calibration()
        print(json.dumps({"roofline_only": shapes}), flush=True)
        return 0
    tok = SyntheticTokenizer(model.args.vocab_size)
    target = Target(model, tok, kv_bits=kv_bits)
    cap = args.block - 1
    W = cap + 1
    rounds_total = args.steps + args.warmup + 2
    max_ctx = args.ctx + W * (rounds_total + 2) + 64
    cache = target.make_cache(max_ctx=max_ctx)
    dcache = drafter.make_cache(max_ctx=max_ctx)
    prompt = np.random.default_rng(1234).integers(0, model.args.vocab_size, args.ctx).tolist()
    t0 = time.time()
    tap = list(dcfg.target_layer_ids)
    logits, fused = model.prefill(prompt, cache, tap)
    drafter.ingest(fused, dcache)
    pending = _pick(logits[0, -1], 0.0)
    torch.cuda.synchronize()
    log(f"prefill {args.ctx} tokens: {time.time() - t0:.1f} s")

    rnd = _DFlashRound(target, drafter, cache, dcache, cap, 0.0, 1.0, 0, 0)
    rnd.pending.fill_(pending)
    for r in range(args.warmup):
        rnd.run(r, use_graph=True)
    torch.cuda.synchronize()
    accepted = []
    t0 = time.perf_counter()
    for r in range(args.steps):
        n, token, _ = rnd.run(args.warmup + r, use_graph=True)
        accepted.append(n + 1)
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    ms_per_step = secs / args.steps * 1e3
    tok_s = sum(accepted) / secs
    mean_accept = sum(accepted) / len(accepted)
    log(f"{args.steps} rounds: {ms_per_step:.3f} ms/round, {tok_s:.1f} accepted tok/s, accept {mean_accept:.2f}")

    # ---- verify step alone: one graph of the 16-row target forward (no advance: idempotent)
    L_now = cache.lengths[0]
    vids = torch.randint(0, model.args.vocab_size, (1, W), dtype=torch.int32, device=model.device)
    vl = torch.empty((W, model.args.vocab_size), dtype=torch.float32, device=model.device)
    vf = torch.empty((W, len(tap) * model.args.hidden_size), dtype=torch.bfloat16, device=model.device)
    model.forward(vids, cache, tap, advance=False, logits_out=vl, fused_out=vf)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        model.forward(vids, cache, tap, advance=False, logits_out=vl, fused_out=vf)
    for _ in range(3):
        g.replay()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s_ev.record()
    for _ in range(args.verify_reps):
        g.replay()
    e_ev.record()
    torch.cuda.synchronize()
    verify_us = s_ev.elapsed_time(e_ev) * 1e3 / args.verify_reps
    kvpt = kv_bytes_per_token(model.args, kv_bits)
    alg_bytes = model.weight_bytes + kvpt * L_now + kvpt * W + W * model.args.vocab_size * 4
    verify_frac = alg_bytes / (verify_us * 1e-6) / (PEAK_HBM_GBS * 1e9)
    log(f"verify step: {verify_us:.1f} us for {alg_bytes / 1e9:.3f} GB algorithmic "
        f"-> {alg_bytes / verify_us / 1e3:.0f} GB/s ({verify_frac * 100:.1f}% of HBM roofline)")

    # ---- dominant kernel: the W8 GEMM, gate_up shape (the largest share of the verify step)
    shapes = gemm_roofline(model, W)
    dom = shapes["gate_up"]
    achieved = dom["bytes"] / dom["us"] / 1e3
    log(f"W8 GEMM per shape: {json.dumps(shapes)}")

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(model.args, 0, args.ctx, W, mean_accept)
        log(f"cpu baseline in {time.time() - t0:.1f} s: {cpu}")

    line = {
        "metric": "accepted tok/s (B=1, Qwen3-8B-shape W8, k=16); verify-step us; % HBM roofline",
        "value": round(tok_s, 2), "unit": "accepted tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random-init W8 weights, seeded 4096-token context)",
        "config": {"workload": "qwen3-8b-shape W8 target + 2-layer DFlash drafter, B=1, "
                               f"{args.ctx}-token context, verify block {W} (k=16), "
                               f"{'8-bit' if kv_bits else 'bf16'} KV, greedy",
                   "global_batch": 1, "seq_len": args.ctx, "parallelism": "single GPU",
                   "weights": "target W8 affine group 64 (bf16 scale/bias); DFlash drafter linears 4-bit "
                              "group 64 (the reference's drafter default)"},
        "accept_len": round(mean_accept, 3),
        "verify_us": round(verify_us, 1),
        "verify_alg_bytes": int(alg_bytes),
        "verify_roofline_frac": round(verify_frac, 4),
        "roofline": {"kernel": "w8_gemm_kernel<1, 2, 2, 8, 1, true> (W8 GEMM, gate_up 24576x4096, M=16, SwiGLU)",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": TRAFFIC_GATE_UP,
                     "bytes_per_launch": dom["bytes"], "us_per_launch": dom["us"], "per_shape": shapes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
