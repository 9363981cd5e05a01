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
  verify17_us  the same at 17 rows (k = 16 drafts + the bonus row), with its roofline fraction
  roofline     the dominant kernel: of the W8 GEMM instantiations the verify forward runs (named
               as a kernel trace names them), the one with the most time per forward; its
               average launch's algorithmic bytes over its average in-graph launch time (one
               launch per layer's weights, HIP events on the launch stream); every instantiation
               with its share is listed under roofline.kernels
  sampled_round_extra_us  the same rounds at temperature 0.6 / top-p 0.95 / top-k 20 (draft
               rows drawn, speculative-sampling acceptance), minus the greedy round time
  acc_us       the standalone acceptance workload [4, 17, 151936] fp32 (T = 1, top-p 0.95),
               graph-replayed, with its HBM roofline fraction
  q06          the Qwen3-0.6B-shaped workload end to end (DSpark block 8, 256 new tokens)
  config_verify  the verify step alone of the other configurations, each against its own
               roofline: Q06 (0.6B shape, 9 rows, 768 context), G12 (Gemma-style 12B shape, 9
               rows, 8192 context, sliding layers reading their 1024-token window) and CB (8B
               shape, 4 rows of 9 over contexts 1024 / 3072 / 6144 / 12288); bf16 KV holding
               seeded random values (timing only), one graph replayed 30 times
  cpu_baseline the CPU oracle (torch, float32 with bf16 rounding points) on the host cores:
               value = accepted tok/s of 5 whole DFlash rounds on the same weights (random
               4096-position context); q06 = the Q06 workload end to end on the same prompt;
               acc = the acceptance workload on every host core, outputs compared with the GPU's
Options for measurements outside the default line: --roofline-only (the GEMM shapes and a copy,
for counter runs), --gemm-sweep M (every plan of the GEMM at the verify shapes), --legs-only,
--acc-only, --verify-eager N.
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
# HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE counter runs of `bench.py --verify-eager 2`
# (profiles/verify_kernels_*_counters.md), per kernel instantiation: the counters' KiB per dispatch
# scaled by what they read for a 256 MiB copy (`bench.py --roofline-only` runs one)
TRAFFIC = {
    # qkv 6144x4096, split-K partials: 13342.68 KiB x 2.000 + 768 KiB
    "w8_gemm_kernel<1, 3, 2, 16, 2, false, 8>": 28112249,
    # o 4096x4096, residual epilogue: 9522.66 KiB x 2.000 + 384 KiB
    "w8_gemm_kernel<1, 1, 2, 16, 3, true, 8>": 19895624,
    # gate_up 24576x4096, SwiGLU: 52846.88 KiB x 2.000 + 384 KiB
    "w8_gemm_kernel<1, 2, 2, 8, 5, false, 8>": 108623626,
    # down 4096x12288, residual epilogue: 27939.95 KiB x 2.000 + 401.78 KiB
    "w8_gemm_kernel<1, 1, 2, 8, 3, false, 8>": 57632436,
    # lm_head 151936x4096, f32 logits: 323501.28 KiB x 2.000 + 9496.38 KiB
    "w8_gemm_kernel<1, 4, 2, 8, 4, false, 8>": 672254912,
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kv_bytes_per_token(args, kv_bits) -> int:
    per_head = args.head_dim * 2 if kv_bits is None else args.head_dim + 4 * (args.head_dim // 64)
    return 2 * per_head * args.num_key_value_heads * args.num_hidden_layers


def gemm_roofline(model, M: int, reps: int = 10):
    """In-graph average launch duration of the W8 GEMM at every verify-step shape, with the
    epilogue and input the forward uses: split-K partials for qkv, the residual-add epilogue for
    o and down, the fused SwiGLU of a normed-later x for gate_up, f32 logits of a normed-later x
    for the head. One CUDA graph per shape holds one launch per layer, each on that layer's
    weights (so every launch streams its weights from HBM), replayed `reps` times between two
    HIP events recorded on the launch stream; the average includes the dispatch gap between
    back-to-back graph kernels, which a kernel trace does not count."""
    import torch
    from mlx_dspark import ops

    dev = model.device
    P, SW, R = ops.DSK_EPI_PARTIAL, ops.DSK_EPI_SWIGLU, ops.DSK_EPI_RESIDUAL
    shapes = {"qkv": ([L.qkv for L in model.layers], P), "o": ([L.o for L in model.layers], R),
              "gate_up": ([L.gate_up for L in model.layers], SW), "down": ([L.down for L in model.layers], R),
              "lm_head": ([model.lm_head], ops.DSK_EPI_STORE)}
    res = {}
    stream = torch.cuda.current_stream()
    eps = model.args.rms_norm_eps
    for name, (ws, epi) in shapes.items():
        K, N = ws[0].K, ws[0].N
        xr = torch.randn(M, K, device=dev).to(torch.bfloat16)
        normed_later = name in ("gate_up", "lm_head")
        x = ops.pack_rn(M=M, K=K, h=xr, norm_w=model.norm, eps=eps) if normed_later else ops.pack(xr)
        h = torch.randn(M, N, device=dev).to(torch.bfloat16)

        def launch(w, y=None):
            if epi == R:
                return ops.w8_residual(x, w, h, next_norm=model.norm, eps=eps)
            out = y if y is not None else (torch.empty(M, N, device=dev, dtype=torch.float32)
                                           if epi == ops.DSK_EPI_STORE else None)
            return ops.w8_gemm(x, w, epi=epi, out=out)

        y = launch(ws[0])
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for w in ws:
                launch(w, None if epi == R else y)
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
        # algorithmic bytes: weights (q + scale/bias) + activation in + output out (the residual
        # epilogue reads and writes h and writes the packed next input)
        out_b = {P: 4 * ops.gemm_splits(M, ws[0].N, K), SW: 1, ops.DSK_EPI_STORE: 4, R: 6}[epi] * M * ws[0].N
        by = ws[0].N * K * 1.0625 + M * K * 2 + out_b
        res[name] = {"us": round(us, 2), "bytes": int(by), "GBs": round(by / us / 1e3, 1), "launches": len(ws),
                     "kernel": ops.gemm_kernel_name(M, ws[0].N, K, epi, normed_later)}
        del g
    return res


def gemm_by_kernel(shapes: dict) -> list:
    """The per-shape timings grouped by the kernel instantiation that runs them, with each
    instantiation's time per verify forward (its shapes' in-graph launch times x launches) and
    share of the GEMM time, largest first. A group's achieved rate is its algorithmic bytes over
    its time per forward: the average launch's bytes over the average launch's duration."""
    groups = {}
    for name, r in shapes.items():
        g = groups.setdefault(r["kernel"], {"kernel": r["kernel"], "shapes": [], "us_per_forward": 0.0,
                                            "bytes_per_forward": 0, "launches_per_forward": 0})
        g["shapes"].append(name)
        g["us_per_forward"] += r["us"] * r["launches"]
        g["bytes_per_forward"] += r["bytes"] * r["launches"]
        g["launches_per_forward"] += r["launches"]
    total = sum(g["us_per_forward"] for g in groups.values())
    out = []
    for g in sorted(groups.values(), key=lambda g: -g["us_per_forward"]):
        achieved = g["bytes_per_forward"] / g["us_per_forward"] / 1e3
        out.append({**g, "us_per_forward": round(g["us_per_forward"], 1), "share": round(g["us_per_forward"] / total, 4),
                    "bytes_per_launch": int(g["bytes_per_forward"] / g["launches_per_forward"]),
                    "us_per_launch": round(g["us_per_forward"] / g["launches_per_forward"], 2),
                    "achieved": round(achieved, 1), "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": TRAFFIC.get(g["kernel"])})
    return out


def gemm_sweep(model, M: int, reps: int = 10) -> dict:
    """Plan sweep of the W8 GEMM at the verify-step shapes through the explicit-plan tuning
    entry (dsk_w8_gemm_rn_planned): every plan it accepts (slab tiles 1-8 dividing the tile
    count, 2- or 4-group batches, 4 / 8 / 16 waves, 1-8 K splits for the partial sums, loads
    pipelined or not), each timed as gemm_roofline times the planner's own (one launch per layer
    on that layer's weights in one graph, HIP events); the planner's choice is marked. The
    planner's rules (w8.hip, plan_gemm) were fitted to sweeps of this kind."""
    import torch
    from mlx_dspark import _hip, ops
    from mlx_dspark._hip import ptr, stream_ptr

    dev = model.device
    P, R, ST = ops.DSK_EPI_PARTIAL, ops.DSK_EPI_RESIDUAL, ops.DSK_EPI_STORE
    SW = model.act_epi
    eps = model.args.rms_norm_eps
    if model.args.sandwich_norms:
        # sandwich norms (the Gemma-style layout): o and down leave split-K partials for the norm
        # that follows them, every projection's x is normed in full
        shapes = {"qkv": ([L.qkv for L in model.layers], P, False), "o": ([L.o for L in model.layers], P, False),
                  "gate_up": ([L.gate_up for L in model.layers], SW, False),
                  "down": ([L.down for L in model.layers], P, False), "lm_head": ([model.lm_head], ST, False)}
    else:
        shapes = {"qkv": ([L.qkv for L in model.layers], P, False), "o": ([L.o for L in model.layers], R, False),
                  "gate_up": ([L.gate_up for L in model.layers], SW, True),
                  "down": ([L.down for L in model.layers], R, False), "lm_head": ([model.lm_head], ST, True)}
    stream = torch.cuda.current_stream()
    out = {}
    for name, (ws, epi, rs) in shapes.items():
        N, K = ws[0].N, ws[0].K
        xr = torch.randn(M, K, device=dev).to(torch.bfloat16)
        x = ops.pack_rn(M=M, K=K, h=xr, norm_w=model.norm, eps=eps) if rs else ops.pack(xr)
        h = torch.randn(M, N, device=dev).to(torch.bfloat16)
        nxt = ops.Packed.empty(M, N, dev, normed_later=True, eps=eps) if epi == R else None
        tiles, G = N // 16, K // 64
        planner = ops.gemm_plan(M, N, K, epi)
        rows = []
        for nt in (1, 2, 3, 4, 6, 8):
            if tiles % nt or (epi == SW and nt % 2):
                continue
            for u in (2, 4):
                for waves in (4, 8, 16):
                    for sk in ((1, 2, 3, 4, 5, 8) if epi == P else (1,)):
                        for pf in (0, 1):
                            plan = (nt, u, waves, sk, pf)
                            if G % u or sk > G // u or waves * ((M + 15) // 16) * nt * 1024 > 65536:
                                continue
                            y = (torch.empty(sk, M, N, device=dev) if epi == P else
                                 torch.empty(M, N, device=dev) if epi == ST else ops.Packed.empty(M, N // 2, dev).data)

                            def launch(w, plan=plan, y=y):
                                _hip.call("dsk_w8_gemm_rn_planned", ptr(x.data), ptr(w.wt), ptr(w.sb), w.bits, M, N, K,
                                          epi, ptr(nxt.data if epi == R else y), ops.DSK_F32 if epi in (P, ST) else ops.DSK_BF16,
                                          N if epi == ST else 0, 0.0, ptr(x.ssq), K // 16 if rs else 0, float(eps),
                                          ptr(h if epi == R else None), N if epi == R else 0, None, 0,
                                          ptr(model.norm if epi == R else None),
                                          ptr(nxt.ssq if epi == R else None), *plan, stream_ptr())
                            try:
                                launch(ws[0])
                                torch.cuda.synchronize()
                            except RuntimeError:            # no compiled kernel for this plan
                                continue
                            g = torch.cuda.CUDAGraph()
                            with torch.cuda.graph(g):
                                for w in ws:
                                    launch(w)
                            g.replay()
                            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                            torch.cuda.synchronize()
                            s_ev.record(stream)
                            for _ in range(reps):
                                g.replay()
                            e_ev.record(stream)
                            torch.cuda.synchronize()
                            us = s_ev.elapsed_time(e_ev) * 1e3 / (reps * len(ws))
                            rows.append({"plan": list(plan), "us": round(us, 2), "planner": plan == tuple(planner)})
                            del g
        rows.sort(key=lambda r: r["us"])
        out[name] = {"N": N, "K": K, "planner_plan": list(planner),
                     "planner_us": next((r["us"] for r in rows if r["planner"]), None),
                     "best": rows[0] if rows else None, "plans": rows}
        log(f"sweep {name} {N}x{K} at M={M}: {len(rows)} plans, best {rows[0] if rows else None}, "
            f"planner {out[name]['planner_us']} us")
    return out


def mall_probe(model, M: int, reps: int = 10) -> dict:
    """The verify GEMMs with their weights in HBM against weights resident in the 256 MB
    memory-side cache: per shape, the in-graph average of 36 launches with the epilogue the
    forward uses, on the 36 layers' weights (`cold`), on one layer's weights 36 times (`same`:
    every launch after the first finds them in the cache) and on two layers' weights in turn
    (`pair`). The gap bounds what prefetching a layer's weights ahead of its GEMM can gain.
    `read` is a plain read of the 36 layers' codes (dsk_prefetch: no arithmetic, no output), the
    fastest of four grid sizes."""
    import torch
    from mlx_dspark import _hip, ops
    from mlx_dspark._hip import ptr, stream_ptr

    P, SW, R = ops.DSK_EPI_PARTIAL, ops.DSK_EPI_SWIGLU, ops.DSK_EPI_RESIDUAL
    eps = model.args.rms_norm_eps
    stream = torch.cuda.current_stream()
    shapes = {"qkv": (lambda L: L.qkv, P), "o": (lambda L: L.o, R), "gate_up": (lambda L: L.gate_up, SW),
              "down": (lambda L: L.down, R)}
    out = {}
    for name, (get, epi) in shapes.items():
        ws_all = [get(L) for L in model.layers]
        K, N = ws_all[0].K, ws_all[0].N
        xr = torch.randn(M, K, device=model.device).to(torch.bfloat16)
        x = (ops.pack_rn(M=M, K=K, h=xr, norm_w=model.norm, eps=eps) if name == "gate_up" else ops.pack(xr))
        h = torch.randn(M, N, device=model.device).to(torch.bfloat16)

        def launch(w):
            if epi == R:
                return ops.w8_residual(x, w, h, next_norm=model.norm, eps=eps)
            return ops.w8_gemm(x, w, epi=epi)

        n = len(ws_all)
        row = {"N": N, "K": K}
        for mode, ws in (("cold", ws_all), ("same", [ws_all[0]] * n), ("pair", [ws_all[i % 2] for i in range(n)])):
            launch(ws[0])
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for w in ws:
                    launch(w)
            for _ in range(2):
                g.replay()
            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            s_ev.record(stream)
            for _ in range(reps):
                g.replay()
            e_ev.record(stream)
            torch.cuda.synchronize()
            row[f"{mode}_us"] = round(s_ev.elapsed_time(e_ev) * 1e3 / (reps * n), 2)
            del g
        # a plain read of the same 36 layers' codes (dsk_prefetch: one launch per layer, no
        # arithmetic, 32 KB in flight per workgroup) at several grid sizes, the fastest kept: the
        # codes are 94 % of a weight's bytes
        sink = torch.zeros(64, dtype=torch.uint8, device=model.device)
        best = None
        for wg in (256, 512, 1024, 2048):
            def read(w, wg=wg):
                _hip.call("dsk_prefetch", ptr(w.wt), w.wt.numel() * w.wt.element_size(), wg, ptr(sink),
                          stream_ptr())

            read(ws_all[0])
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for w in ws_all:
                    read(w)
            g.replay()
            s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            s_ev.record(stream)
            for _ in range(reps):
                g.replay()
            e_ev.record(stream)
            torch.cuda.synchronize()
            us = round(s_ev.elapsed_time(e_ev) * 1e3 / (reps * n), 2)
            del g
            if best is None or us < best[0]:
                best = (us, wg)
        row["read_us"], row["read_workgroups"] = best
        row["read_TBs"] = round(ws_all[0].wt.numel() * ws_all[0].wt.element_size() / best[0] / 1e6, 2)
        out[name] = row
        log(f"memory-side cache probe {name} {N}x{K}: {row}")
    # the same read over the logits head's codes, one launch: the streaming rate without the
    # per-launch ramp and tail weighing on it
    w = model.lm_head
    nbytes = w.wt.numel() * w.wt.element_size()
    best = None
    for wg in (512, 1024, 2048, 4096):
        _hip.call("dsk_prefetch", ptr(w.wt), nbytes, wg, ptr(sink), stream_ptr())
        torch.cuda.synchronize()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record(stream)
        for _ in range(reps):
            _hip.call("dsk_prefetch", ptr(w.wt), nbytes, wg, ptr(sink), stream_ptr())
        e_ev.record(stream)
        torch.cuda.synchronize()
        us = round(s_ev.elapsed_time(e_ev) * 1e3 / reps, 2)
        if best is None or us < best[0]:
            best = (us, wg)
    out["head_read"] = {"bytes": nbytes, "us": best[0], "workgroups": best[1],
                        "TBs": round(nbytes / best[0] / 1e6, 2)}
    log(f"memory-side cache probe: plain read of the head's codes {out['head_read']}")
    # the cost of a launch itself: 100 launches of a one-workgroup kernel with one load and one
    # store (dsk_lens_add on one length) in one graph
    lens = torch.zeros(1, dtype=torch.int32, device=model.device)
    ops.lens_add(lens, None, 1)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(100):
            ops.lens_add(lens, None, 1)
    g.replay()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s_ev.record(stream)
    for _ in range(reps):
        g.replay()
    e_ev.record(stream)
    torch.cuda.synchronize()
    out["launch_us"] = round(s_ev.elapsed_time(e_ev) * 1e3 / (reps * 100), 2)
    del g
    log(f"memory-side cache probe: one tiny kernel in a graph {out['launch_us']} us per launch")
    return out


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
    word.zero_()                                  # offset 0: the outputs the CPU leg reproduces
    run()
    return {"us": round(us, 2), "bytes": int(nbytes), "GBs": round(nbytes / us / 1e3, 1),
            "roofline_frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
            "config": "B=4, 16 drafts + bonus, V=151936 fp32, T=1, top_p=0.95, top_k=0",
            "n": n.tolist(), "token": tok.tolist()}


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


def _cores() -> int:
    return len(os.sched_getaffinity(0))


def cpu_q8_rounds(model, drafter, dcfg, ctx: int, cap: int, kv_bits, rounds: int = 5):
    """The oracle (torch on the host CPU, float32 with bf16 rounding points) running whole
    greedy DFlash rounds on the bench's own target and drafter weights: drafter block over its
    context, a 16-row verify of all 36 layers over a ctx-position 8-bit KV context, acceptance
    and rollback. Both the target's KV and the drafter's context hold seeded random rows (an
    oracle prefill of the 4096-token prompt would take hours on the CPU); one warm-up round,
    then ``rounds`` timed rounds."""
    import torch

    from oracle import model as OM
    from oracle import spec as SP

    torch.set_num_threads(_cores())
    t0 = time.perf_counter()
    tgt = OM.OracleTarget(model, kv_bits=kv_bits)
    od = OM.OracleDFlash(drafter, tgt)
    build_s = time.perf_counter() - t0
    a = model.args
    g = torch.Generator().manual_seed(5)
    for l in range(len(tgt.layers)):
        tgt.K[l] = OM.bf(torch.randn(ctx, a.num_key_value_heads, a.head_dim, generator=g))
        tgt.V[l] = OM.bf(torch.randn(ctx, a.num_key_value_heads, a.head_dim, generator=g))
    tgt.offset = ctx
    c = dcfg
    for l in range(len(od.layers)):
        od.K[l] = OM.bf(torch.randn(ctx, c.num_key_value_heads, c.head_dim, generator=g))
        od.V[l] = OM.bf(torch.randn(ctx, c.num_key_value_heads, c.head_dim, generator=g))
    tap = list(c.target_layer_ids)
    new_ctx = OM.bf(torch.randn(1, len(tap) * a.hidden_size, generator=g))
    pending = 1
    times, accepted = [], []
    for r in range(rounds + 1):
        t0 = time.perf_counter()
        n, token, drafts, new_ctx = SP.dflash_round(tgt, od, pending, new_ctx, cap, tap, int(c.mask_token_id),
                                                     int(c.block_size))
        dt = time.perf_counter() - t0
        pending = token
        if r:
            times.append(dt)
            accepted.append(n + 1)
    # the verify forward alone, three times (rolled back each time)
    vt = []
    for _ in range(3):
        ids = torch.randint(0, a.vocab_size, (cap + 1,), generator=g).tolist()
        t0 = time.perf_counter()
        tgt.forward(ids, tap)
        vt.append(time.perf_counter() - t0)
        tgt.trim(cap + 1)
    secs = sum(times)
    return {"value": round(sum(accepted) / secs, 4), "unit": "accepted tok/s", "cores": _cores(), "kind": "port",
            "sample": (f"oracle (torch fp32, bf16 rounding points): {rounds} whole greedy DFlash rounds after one "
                       f"warm-up on the bench's weights (36-layer target verify of {cap + 1} rows over a "
                       f"{ctx}-position {'8-bit' if kv_bits else 'bf16'} KV context of seeded random rows, "
                       f"2-layer drafter block, 151936-row heads), {secs:.1f} s of CPU work; median round "
                       f"{statistics.median(times) * 1e3:.0f} ms, mean accept length "
                       f"{sum(accepted) / len(accepted):.2f}; build (dequantize to fp32) {build_s:.0f} s"),
            "round_ms": round(statistics.median(times) * 1e3, 1),
            "verify_ms": round(statistics.median(vt) * 1e3, 1)}


def q06_models(seed: int = 6):
    """The Qwen3-0.6B-shaped W8 target and its 1-layer DSpark drafter (taps 1, 14, 27,
    block 8), kept with their MLX-layout codes for the oracle."""
    from mlx_dspark import synthetic
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer

    model = synthetic.build_target("qwen3-0.6b", seed=seed, keep_mlx=True)
    d, cfg = synthetic.build_dspark(model.args, seed=seed + 1, keep_mlx=True, num_hidden_layers=1, block_size=8,
                                    taps=[1, 14, 27])
    tok = SyntheticTokenizer(model.args.vocab_size)
    return Target(model, tok), tok, d, cfg


Q06_PROMPT, Q06_NEW = 512, 256


def q06_gpu(target, tok, d) -> dict:
    """Q06 end to end on the GPU: greedy DSpark decoding, block 8 (8 drafts verified per round,
    W = 9), lookup drafts off, 256 new tokens after a 512-token prompt; one untimed run first
    (graph capture), then one timed run."""
    import numpy as np

    from mlx_dspark.generate import speculative_generate
    prompt = np.random.default_rng(512).integers(0, target.model.args.vocab_size, Q06_PROMPT).tolist()
    kw = dict(prompt_ids=prompt, max_new_tokens=Q06_NEW, max_draft_tokens=8, lookup_drafts=False)
    speculative_generate(target, tok, d, **kw)
    res = speculative_generate(target, tok, d, **kw)
    return {"tok_s": round(res.num_tokens / res.seconds, 1), "accept_len": round(res.mean_accept_len, 3),
            "tokens": res.token_ids, "seconds": round(res.seconds, 4), "prompt": prompt}


def cpu_q06(target, d, cfg, prompt) -> dict:
    """Q06 end to end on the oracle: the same prompt, drafter and settings as ``q06_gpu``."""
    import torch

    from oracle import model as OM
    from oracle import spec as SP

    torch.set_num_threads(_cores())
    tgt, od = OM.OracleTarget(target.model), OM.OracleDSpark(d)
    t0 = time.perf_counter()
    toks, accepts = SP.dspark_generate(tgt, od, prompt, Q06_NEW, 8, list(cfg.target_layer_ids),
                                       int(cfg.mask_token_id), int(cfg.block_size))
    secs = time.perf_counter() - t0
    return {"tok_s": round(len(toks) / secs, 2), "accept_len": round(len(toks) / max(1, len(accepts)), 3),
            "seconds": round(secs, 1), "tokens": toks}


def q06_teacher_forced(target, prompt, tokens) -> dict:
    """The oracle's verdict on the GPU's Q06 stream: one oracle forward over prompt + stream
    (teacher forcing); how many GPU tokens are the oracle's argmax, and the largest gap between
    the oracle's best RMS-normalised logit and the GPU token's."""
    from oracle import model as OM
    logits, _ = OM.OracleTarget(target.model).forward(list(prompt) + list(tokens[:-1]))
    rows = logits[len(prompt) - 1:]
    rn = rows / rows.pow(2).mean(-1, keepdim=True).sqrt()
    import torch
    t = torch.tensor(tokens)
    gap = (rn.max(-1).values - rn.gather(1, t[:, None])[:, 0])
    return {"oracle_argmax": int((gap == 0).sum()), "of": len(tokens), "max_gap": round(float(gap.max()), 4)}


# The other benchmark configurations' verify steps, timed alone: (name, synthetic shape, context
# per batch row, rows per batch row, the configuration's 70 %-of-roofline bound in us)
CONFIG_LEGS = [
    ("Q06", "qwen3-0.6b", [768], 9, 129.0),
    ("G12", "gemma-12b", [8192], 9, 2388.0),
    ("CB", "qwen3-8b", [1024, 3072, 6144, 12288], 9, 2029.0),
]


def verify_leg(shape: str, lens: list, W: int, reps: int = 30) -> dict:
    """One graph-replayed verify forward of `shape` (B = len(lens) rows of W new tokens each over
    contexts `lens`, bf16 KV holding seeded N(0, 1) values: a timing-only context, no prefill),
    HIP events around `reps` replays. Algorithmic bytes: the W8 weights, each layer's visible K/V
    of every row (a sliding layer at most its window), the new rows' K/V writes and the fp32
    logits."""
    import torch

    from mlx_dspark import synthetic

    model = synthetic.build_target(shape, seed=0)
    a = model.args
    B = len(lens)
    cache = model.make_cache(B=B, max_ctx=max(lens) + W + 64)
    g = torch.Generator(device=model.device).manual_seed(5)
    for l in range(a.num_hidden_layers):
        cache.k[l].normal_(generator=g)
        cache.v[l].normal_(generator=g)
    cache.set_lengths(lens)
    ids = torch.randint(0, a.vocab_size, (B, W), dtype=torch.int32, device=model.device, generator=g)
    model.forward(ids, cache, None, advance=False)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        model.forward(ids, cache, None, advance=False)
    for _ in range(3):
        graph.replay()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s_ev.record()
    for _ in range(reps):
        graph.replay()
    e_ev.record()
    torch.cuda.synchronize()
    us = s_ev.elapsed_time(e_ev) * 1e3 / reps
    per_tok = 2 * a.num_key_value_heads * a.head_dim * 2          # K and V, bf16, one layer
    kv_read = sum(min(L + W, a.window(l) or (L + W)) * per_tok for l in range(a.num_hidden_layers) for L in lens)
    kv_write = B * W * per_tok * a.num_hidden_layers
    alg = model.weight_bytes + kv_read + kv_write + B * W * a.vocab_size * 4
    out = {"verify_us": round(us, 1), "alg_bytes": int(alg),
           "roofline_frac": round(alg / (us * 1e-6) / (PEAK_HBM_GBS * 1e9), 4),
           "rows": B * W, "contexts": lens, "kv": "bf16 (seeded random values)"}
    del graph, cache, model
    torch.cuda.empty_cache()
    return out


def cpu_acc(gpu_out=None, reps: int = 3) -> dict:
    """The acceptance oracle (C; its (row, position) items spread over the host cores with OpenMP)
    on the standalone acceptance workload: median of ``reps`` runs; outputs compared with the GPU's
    on the same inputs and Philox (seed, offset)."""
    from oracle import accept as A
    p, q, draft = (t.numpy() for t in acc_inputs())
    times, res = [], None
    for _ in range(reps):
        t0 = time.perf_counter()
        res = A.accept_sample(p, q, draft, 1.0, 0.95, 0, seed=7, offset=0)
        times.append(time.perf_counter() - t0)
    out = {"ms": round(statistics.median(times) * 1e3, 1), "cores": A.threads()}
    if gpu_out is not None:
        out["bit_exact_vs_gpu"] = bool(list(res["n"]) == gpu_out["n"] and list(res["token"]) == gpu_out["token"])
    return out


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
    ap.add_argument("--no-config-legs", action="store_true",
                    help="skip the Q06 / G12 / CB verify-step timings")
    ap.add_argument("--legs-only", action="store_true",
                    help="only the Q06 / G12 / CB verify-step timings (one JSON line)")
    ap.add_argument("--verify-reps", type=int, default=50)
    ap.add_argument("--roofline-only", action="store_true",
                    help="build the target, time the W8 GEMM shapes and a 256 MiB copy only (counter runs)")
    ap.add_argument("--acc-only", action="store_true",
                    help="time the standalone acceptance workload [4, 17, 151936] only")
    ap.add_argument("--mall-probe", action="store_true",
                    help="build the target and time the verify GEMMs with their weights in HBM and "
                         "resident in the memory-side cache (one JSON line)")
    ap.add_argument("--gemm-sweep", type=int, default=0, metavar="M",
                    help="build the target and sweep the W8 GEMM plans at the verify shapes for M rows (one JSON line)")
    ap.add_argument("--verify-eager", type=int, default=0, metavar="N",
                    help="build the target, prefill the context, run N eager verify forwards and exit "
                         "(one kernel launch per op: for counter collection)")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this engine has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from mlx_dspark import ops, synthetic
    from mlx_dspark.generate import _DFlashPipe, _pick
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer

    kv_bits = args.kv_bits or None
    torch.cuda.init()
    if args.acc_only:
        print(json.dumps({"acc": acc_timing()}), flush=True)
        return 0
    if args.legs_only:
        legs = {}
        for name, shape, lens, w, bound in CONFIG_LEGS:
            legs[name] = verify_leg(shape, lens, w)
            legs[name]["baseline_bound_us"] = bound
            log(f"{name} verify: {legs[name]['verify_us']} us, {legs[name]['roofline_frac'] * 100:.1f}% of roofline")
        print(json.dumps({"config_verify": legs}), flush=True)
        return 0
    t_build = time.time()
    keep = not args.no_cpu_baseline            # the oracle reads the MLX-layout codes
    model = synthetic.build_target(args.target, seed=0, keep_mlx=keep and not args.gemm_sweep)
    if args.mall_probe:
        print(json.dumps({"mall_probe": {"target": args.target, "M": args.block,
                                         "shapes": mall_probe(model, args.block)}}), flush=True)
        return 0
    if args.gemm_sweep:
        log(f"built {args.target} W8 target ({model.weight_bytes / 1e9:.2f} GB) in {time.time() - t_build:.1f} s")
        print(json.dumps({"gemm_sweep": {"target": args.target, "M": args.gemm_sweep,
                                         "shapes": gemm_sweep(model, args.gemm_sweep)}}), flush=True)
        return 0
    if args.verify_eager:
        # seeded random context written straight into the KV pools (no prefill), then eager
        # verify forwards of --block rows: every op is its own launch (for counter collection,
        # any --target; the hidden-state taps a 5-tap drafter would read)
        from mlx_dspark.synthetic import evenly_spaced_layers
        W = args.block
        target = Target(model, SyntheticTokenizer(model.args.vocab_size), kv_bits=kv_bits)
        cache = target.make_cache(max_ctx=args.ctx + W + 64)
        tap = list(evenly_spaced_layers(model.args.num_hidden_layers, 5))
        g = torch.Generator(device=model.device).manual_seed(4)
        for l in range(model.args.num_hidden_layers):
            for pool, sb in ((cache.k[l], cache.k_sb[l]), (cache.v[l], cache.v_sb[l])):
                if sb is None:
                    pool.copy_(torch.randn(pool.shape, generator=g, device=model.device).to(pool.dtype))
                else:
                    pool.copy_(torch.randint(0, 256, pool.shape, generator=g, device=model.device).to(pool.dtype))
                    sb.fill_(0x3C23 | (0xBF80 << 16) - (1 << 32))     # scale bf16(0.01), bias bf16(-1)
        cache.set_lengths([args.ctx])
        vids = torch.randint(0, model.args.vocab_size, (1, W), dtype=torch.int32, device=model.device)
        for _ in range(args.verify_eager):
            model.forward(vids, cache, tap, advance=False)
        torch.cuda.synchronize()
        print(json.dumps({"verify_eager": args.verify_eager, "target": args.target, "rows": W,
                          "context": cache.lengths[0]}), flush=True)
        return 0
    drafter, dcfg = synthetic.build_dflash(model.args, seed=1, block_size=args.block, n_taps=5, bits=4, keep_mlx=keep)
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
    rounds_total = 2 * (args.steps + max(args.warmup, 4)) + 2  # greedy rounds, then sampled rounds
    max_ctx = args.ctx + W * (rounds_total + 2) + 64
    cache = target.make_cache(max_ctx=max_ctx)
    dcache = drafter.make_cache(max_ctx=max_ctx)
    prompt = np.random.default_rng(1234).integers(0, model.args.vocab_size, args.ctx).tolist()
    t0 = time.time()
    tap = list(dcfg.target_layer_ids)
    # the prompt's dense prefill (layer by layer over all rows), timed after a short warm-up
    # prefill that settles the library GEMM's plans; the weights' bf16 rows are held in HBM
    # (expanded once here, as a server does at load), so the prefill multiplies them directly
    dense_held = model.keep_dense_weights()
    log(f"dense prefill weights held as bf16 rows: {dense_held / 1e9:.2f} GB")
    wc = target.make_cache(max_ctx=1024)
    model.prefill(prompt[:512], wc, tap)
    del wc
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits, fused = model.prefill(prompt, cache, tap)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3
    a_ = model.args
    lin_params = sum(L.qkv.N * L.qkv.K + L.o.N * L.o.K + L.gate_up.N * L.gate_up.K + L.down.N * L.down.K
                     for L in model.layers)
    attn_flop = 4 * a_.num_attention_heads * a_.head_dim * a_.num_hidden_layers * args.ctx * (args.ctx + 1) / 2
    prefill_flop = 2 * args.ctx * lin_params + attn_flop
    log(f"prefill {args.ctx} tokens (dense): {prefill_ms:.1f} ms, {prefill_flop / prefill_ms / 1e9:.0f} TFLOP/s")
    drafter.ingest(fused, dcache)
    pending = _pick(logits[0, -1], 0.0)
    torch.cuda.synchronize()

    # rounds as dflash_generate runs them: each enqueued before the host reads the previous
    # round's ids (two alternating graph-replayed round objects)
    pipe = _DFlashPipe(target, drafter, cache, dcache, cap, 0.0, 1.0, 0, 0)
    pipe.start(pending)
    for r in range(max(args.warmup, 4)):       # both round objects captured before the timing
        pipe.enqueue()
        pipe.collect()
    torch.cuda.synchronize()
    accepted = []
    t0 = time.perf_counter()
    pipe.enqueue()
    for r in range(args.steps):
        if r + 1 < args.steps:
            pipe.enqueue()
        n, token, _ = pipe.collect()
        accepted.append(n + 1)
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    ms_per_step = secs / args.steps * 1e3
    tok_s = sum(accepted) / secs
    mean_accept = sum(accepted) / len(accepted)
    log(f"{args.steps} rounds: {ms_per_step:.3f} ms/round, {tok_s:.1f} accepted tok/s, accept {mean_accept:.2f}")

    # ---- the same rounds sampled (T 0.6, top-p 0.95, top-k 20: draft rows drawn, speculative
    # sampling acceptance), graph-replayed: the extra time per round over greedy
    spipe = _DFlashPipe(target, drafter, cache, dcache, cap, 0.6, 0.95, 20, 5)
    spipe.start(token)
    for r in range(max(args.warmup, 4)):
        spipe.enqueue()
        spipe.collect()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    spipe.enqueue()
    for r in range(args.steps):
        if r + 1 < args.steps:
            spipe.enqueue()
        spipe.collect()
    torch.cuda.synchronize()
    sampled_ms = (time.perf_counter() - t0) / args.steps * 1e3
    log(f"sampled rounds: {sampled_ms:.3f} ms/round (+{(sampled_ms - ms_per_step) * 1e3:.0f} us over greedy)")

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

    # ---- the same verify step at W = 17 (k = 16 drafts + the bonus row)
    W17 = W + 1
    vids17 = torch.randint(0, model.args.vocab_size, (1, W17), dtype=torch.int32, device=model.device)
    model.forward(vids17, cache, tap, advance=False)
    g17 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g17):
        model.forward(vids17, cache, tap, advance=False)
    for _ in range(3):
        g17.replay()
    torch.cuda.synchronize()
    s_ev.record()
    for _ in range(args.verify_reps):
        g17.replay()
    e_ev.record()
    torch.cuda.synchronize()
    verify17_us = s_ev.elapsed_time(e_ev) * 1e3 / args.verify_reps
    alg17 = model.weight_bytes + kvpt * L_now + kvpt * W17 + W17 * model.args.vocab_size * 4
    verify17_frac = alg17 / (verify17_us * 1e-6) / (PEAK_HBM_GBS * 1e9)
    del g17
    log(f"verify step at W = {W17}: {verify17_us:.1f} us ({verify17_frac * 100:.1f}% of HBM roofline)")

    # ---- overlap experiment: the same 16-row verify with each layer's o and gate|up weights read
    # on a side stream during its attention stage (Qwen3W8.prefetch_weights); same logits
    model.prefetch_weights(True)
    vlp = torch.empty_like(vl)
    model.forward(vids, cache, tap, advance=False, logits_out=vlp, fused_out=vf)
    gp = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gp):
        model.forward(vids, cache, tap, advance=False, logits_out=vlp, fused_out=vf)
    for _ in range(3):
        gp.replay()
    torch.cuda.synchronize()
    s_ev.record()
    for _ in range(args.verify_reps):
        gp.replay()
    e_ev.record()
    torch.cuda.synchronize()
    verify_prefetch_us = s_ev.elapsed_time(e_ev) * 1e3 / args.verify_reps
    g.replay()
    torch.cuda.synchronize()
    prefetch_same = bool(torch.equal(vl, vlp))
    del gp
    model.prefetch_weights(False)
    log(f"verify step with the o / gate_up weights prefetched on a side stream: {verify_prefetch_us:.1f} us "
        f"(logits identical: {prefetch_same})")

    # ---- the dominant kernel: of the W8 GEMM instantiations the verify step runs, the one with
    # the most time per forward (in-graph launch times x launches per forward)
    shapes = gemm_roofline(model, W)
    kernels = gemm_by_kernel(shapes)
    dom = kernels[0]
    achieved = dom["achieved"]
    log(f"W8 GEMM per shape: {json.dumps(shapes)}")
    log(f"W8 GEMM per kernel: {json.dumps(kernels)}")

    # ---- standalone acceptance workload and the Q06 end-to-end workload on the GPU
    acc = acc_timing()
    log(f"acceptance [4, 17, 151936]: {acc['us']} us ({acc['roofline_frac'] * 100:.1f}% of HBM roofline)")
    q_target, q_tok, q_d, q_cfg = q06_models()
    q06 = q06_gpu(q_target, q_tok, q_d)
    log(f"qwen3-0.6b DSpark k=8 end to end: {q06['tok_s']} tok/s, accept {q06['accept_len']}")

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_q8_rounds(model, drafter, dcfg, args.ctx, cap, kv_bits)
        log(f"cpu baseline, Q8 rounds in {time.time() - t0:.1f} s: {cpu['value']} tok/s")
        t0 = time.time()
        cq = cpu_q06(q_target, q_d, q_cfg, q06["prompt"])
        same = 0
        while same < min(len(cq["tokens"]), len(q06["tokens"])) and cq["tokens"][same] == q06["tokens"][same]:
            same += 1
        tf = q06_teacher_forced(q_target, q06["prompt"], q06["tokens"])
        cpu["q06"] = {"tok_s": cq["tok_s"], "accept_len": cq["accept_len"], "seconds": cq["seconds"],
                      "tokens_equal_to_gpu": same, "gpu_stream_teacher_forced": tf}
        log(f"cpu baseline, Q06 end to end in {time.time() - t0:.1f} s: {cq['tok_s']} tok/s, "
            f"{same} leading tokens equal to the GPU's; GPU stream under the oracle: {tf}")
        t0 = time.time()
        cpu["acc"] = cpu_acc({"n": acc["n"], "token": acc["token"]})
        log(f"cpu baseline, acceptance in {time.time() - t0:.1f} s: {cpu['acc']}")

    legs = {}
    if not args.no_config_legs:
        for name, shape, lens, w, bound in CONFIG_LEGS:
            try:
                legs[name] = verify_leg(shape, lens, w)
                legs[name]["baseline_bound_us"] = bound
                log(f"{name} verify ({shape}, rows {len(lens)}x{w}, contexts {lens}): {legs[name]['verify_us']} us, "
                    f"{legs[name]['roofline_frac'] * 100:.1f}% of HBM roofline (the configuration's 70% bound {bound} us)")
            except Exception as e:                      # a leg never takes the headline line down
                legs[name] = {"error": f"{type(e).__name__}: {e}"}
                log(f"{name} verify leg failed: {legs[name]['error']}")

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
        "sampled_round_ms": round(sampled_ms, 4),
        "sampled_round_extra_us": round((sampled_ms - ms_per_step) * 1e3, 1),
        "verify_us": round(verify_us, 1),
        "verify_alg_bytes": int(alg_bytes),
        "verify_roofline_frac": round(verify_frac, 4),
        "prefill_ms": round(prefill_ms, 1),
        "prefill_tflops": round(prefill_flop / prefill_ms / 1e9, 1),
        "prefill_weights": f"bf16 rows held in HBM ({dense_held / 1e9:.1f} GB, expanded once before the timing)",
        "verify17_us": round(verify17_us, 1),
        "verify17_alg_bytes": int(alg17),
        "verify17_roofline_frac": round(verify17_frac, 4),
        "verify_prefetch_us": round(verify_prefetch_us, 1),
        "verify_prefetch": "the 16-row verify with each layer's o and gate|up weights read on a side stream during "
                           f"its attention stage (overlap experiment, off in the engine); logits identical: {prefetch_same}",
        "roofline": {"kernel": f"{dom['kernel']} (W8 GEMM: {' and '.join(dom['shapes'])} of the {W}-row verify, "
                               f"{dom['share'] * 100:.1f}% of its GEMM time)",
                     "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": TRAFFIC.get(dom["kernel"]),
                     "bytes_per_launch": dom["bytes_per_launch"], "us_per_launch": dom["us_per_launch"],
                     "kernels": kernels, "per_shape": shapes},
        "acc_us": acc["us"],
        "acc_roofline_frac": acc["roofline_frac"],
        "acc": {k: v for k, v in acc.items() if k not in ("n", "token")},
        "q06": {"tok_s": q06["tok_s"], "accept_len": q06["accept_len"],
                "config": "qwen3-0.6b-shape W8 + 1-layer DSpark (taps 1, 14, 27), prompt 512, block 8, greedy, "
                          "256 new tokens, bf16 KV"},
        "config_verify": legs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
