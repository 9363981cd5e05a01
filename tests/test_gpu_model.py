"""GPU parity of the whole verify path on small synthetic W8 models: target forward with
hidden-state tap (bf16 and 8-bit KV), KV rollback, the DFlash drafter, and greedy
speculative decoding reproducing the oracle's greedy token stream."""

import numpy as np
import pytest
import torch

from _parity import Twin, check_logits, check_greedy_stream
from oracle import model as OM

pytestmark = pytest.mark.gpu
MIN_MATCH = 8      # leading greedy tokens that must equal the oracle's
TOL = 2e-2   # greedy-stream margin rule (normalised logits)


@pytest.fixture(scope="module")
def tiny(dev):
    from mlx_dspark import synthetic
    return synthetic.build_target("tiny", seed=3, keep_mlx=True)


@pytest.mark.parametrize("kv_bits", [None, 8])
def test_target_forward_tap_and_rollback(dev, tiny, kv_bits):
    print(f"target forward kv_bits={kv_bits}", flush=True)
    model = tiny
    V = model.args.vocab_size
    rng = np.random.default_rng(0)
    prompt = rng.integers(0, V, 70).tolist()
    tap = [0, 2]
    cache = model.make_cache(max_ctx=256, kv_bits=kv_bits)
    logits, fused = model.prefill(prompt, cache, tap)
    ref = Twin(lambda: OM.OracleTarget(model, kv_bits=kv_bits))
    (rl, rf), (el, _) = ref.forward(prompt, tap)
    check_logits(logits[0, -1], rl[-1], "prefill last row", exact=el[-1])
    assert fused.shape == (1, 70, 2 * model.args.hidden_size)
    assert (fused[0].float().cpu() - rf).abs().max() < 0.05 * rf.abs().max()
    # verify block of 9 rows, advance=False, then roll back to n = 3 accepted
    block = rng.integers(0, V, 9).tolist()
    ids = torch.tensor([block], dtype=torch.int32, device=dev)
    vl, vf = model.forward(ids, cache, tap, advance=False)
    (rvl, _), (evl, _) = ref.forward(block, tap)
    check_logits(vl[0], rvl, "verify block", exact=evl)
    n = torch.tensor([3], dtype=torch.int32, device=dev)
    from mlx_dspark import ops
    ops.lens_add(cache.seq_lens, n, 1)
    cache.note_lengths([70 + 4])
    ref.trim(9 - 4)
    nxt = rng.integers(0, V, 5).tolist()
    l2, _ = model.forward(torch.tensor([nxt], dtype=torch.int32, device=dev), cache, None)
    (r2, _), (e2, _) = ref.forward(nxt)
    check_logits(l2[0], r2, "after rollback", exact=e2)
    assert int(cache.seq_lens.item()) == 70 + 4 + 5


def test_tied_head_and_target_run_api(dev):
    from mlx_dspark import synthetic
    from mlx_dspark.target import Target
    model = synthetic.build_target("tiny-tied", seed=5, keep_mlx=True)
    t = Target(model, None)
    t.verify_tap()
    cache = t.make_cache(max_ctx=128)
    ids = [[5, 6, 7, 8, 9]]
    lg, fu = t.run(ids, cache, [1])
    (rl, _), (el, _) = Twin(lambda: OM.OracleTarget(model)).forward(ids[0], [1])
    check_logits(lg[0], rl, "tied head", exact=el)
    assert cache[0].offset == 5
    for c in cache:                        # the reference's per-layer trim loop trims once
        c.trim(2)
    assert cache.offset == 3 and int(cache.seq_lens.item()) == 3


def test_dflash_drafter_matches_oracle(dev, tiny):
    from mlx_dspark import synthetic
    d, cfg = synthetic.build_dflash(tiny.args, seed=9, keep_mlx=True, num_hidden_layers=2, block_size=8, n_taps=2)
    d.bind(tiny)
    rng = np.random.default_rng(1)
    V = tiny.args.vocab_size
    prompt = rng.integers(0, V, 40).tolist()
    cache = tiny.make_cache(max_ctx=256)
    _, fused = tiny.prefill(prompt, cache, list(cfg.target_layer_ids))
    dcache = d.make_cache(max_ctx=256)
    block = [int(prompt[-1])] + [cfg.mask_token_id] * (cfg.block_size - 1)
    got = d(block, fused[0], dcache, logits_start=1)
    ref_t = OM.OracleTarget(tiny)
    oa = Twin(lambda: OM.OracleDFlash(d, ref_t))
    want, ex = oa(block, fused[0].float().cpu(), logits_start=1)
    check_logits(got[0], want, "dflash round 1", exact=ex)
    # a second round: 3 more context rows
    more = fused[0, :3]
    got2 = d(block, more, dcache, logits_start=1)
    want2, ex2 = oa(block, more.float().cpu(), logits_start=1)
    check_logits(got2[0], want2, "dflash round 2", exact=ex2)


def test_dflash_sliding_window_drafter_matches_oracle(dev, tiny):
    """DFlash sliding-window layers (src/mlx_dspark/dflash_model.py:103-109, :128-132, :186-195):
    layer 0 slides with a 6-position window (block queries see keys P - 5 .. P, the block causal
    inside it), layer 1 attends to everything. Two rounds against the oracle; an oracle whose
    window is longer differs from the GPU by more than the bound (the window is live)."""
    import dataclasses
    from mlx_dspark import synthetic
    print("dflash sliding window 6", flush=True)
    d, cfg = synthetic.build_dflash(tiny.args, seed=11, keep_mlx=True, num_hidden_layers=2, block_size=8, n_taps=2,
                                    layer_types=("sliding_attention", "full_attention"), sliding_window=6)
    d.bind(tiny)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, tiny.args.vocab_size, 40).tolist()
    cache = tiny.make_cache(max_ctx=256)
    _, fused = tiny.prefill(prompt, cache, list(cfg.target_layer_ids))
    dcache = d.make_cache(max_ctx=256)
    block = [int(prompt[-1])] + [cfg.mask_token_id] * (cfg.block_size - 1)
    ref_t = OM.OracleTarget(tiny)
    oa = Twin(lambda: OM.OracleDFlash(d, ref_t))
    wide = OM.OracleDFlash(d, ref_t)
    wide.c = dataclasses.replace(wide.c, sliding_window=12)
    ctx = fused[0].float().cpu()
    got = d(block, fused[0], dcache, logits_start=1)
    want, ex = oa(block, ctx, logits_start=1)
    bound = check_logits(got[0], want, "sliding round 1", exact=ex)
    mx, _ = OM.logit_diff(got[0], wide(block, ctx, logits_start=1))
    print(f"oracle with a 12-position window: normalised max-abs {mx:.4f}", flush=True)
    assert mx > bound
    more = fused[0, :3]
    got2 = d(block, more, dcache, logits_start=1)
    want2, ex2 = oa(block, more.float().cpu(), logits_start=1)
    check_logits(got2[0], want2, "sliding round 2", exact=ex2)


@pytest.mark.parametrize("use_graph", [False, True])
def test_dflash_generate_reproduces_greedy_stream(dev, tiny, use_graph):
    from mlx_dspark import synthetic
    from mlx_dspark.generate import dflash_generate
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    d, cfg = synthetic.build_dflash(tiny.args, seed=9, keep_mlx=True, num_hidden_layers=2, block_size=8, n_taps=2)
    d.bind(tiny)
    tok = SyntheticTokenizer(tiny.args.vocab_size)
    target = Target(tiny, tok)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, tiny.args.vocab_size, 33).tolist()
    res = dflash_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=24, use_graph=use_graph)
    check_greedy_stream(tiny, prompt, res.token_ids, MIN_MATCH)
    assert res.num_tokens >= 24 and sum(res.accept_lengths) + 1 == res.num_tokens
    assert res.text == tok.decode(res.token_ids)


class _CyclingCap:
    """A duck-typed cap controller (calibrate.py CapController's .cap / .update): cycles through
    caps and records every update."""

    def __init__(self, caps):
        self.caps, self.i, self.updates = list(caps), 0, []

    @property
    def cap(self):
        return self.caps[self.i % len(self.caps)]

    def update(self, n_accepted, n_drafted):
        self.updates.append((n_accepted, n_drafted))
        self.i += 1


def test_dflash_generate_with_cap_controller(dev, tiny):
    """The cap is re-read every round (generate.py:537-538): verify widths vary, the greedy
    stream still equals greedy decoding, and update() sees (accepted, drafted) per round."""
    from mlx_dspark import synthetic
    from mlx_dspark.generate import dflash_generate
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    d, cfg = synthetic.build_dflash(tiny.args, seed=9, keep_mlx=True, num_hidden_layers=2, block_size=8, n_taps=2)
    d.bind(tiny)
    tok = SyntheticTokenizer(tiny.args.vocab_size)
    target = Target(tiny, tok)
    prompt = np.random.default_rng(4).integers(0, tiny.args.vocab_size, 29).tolist()
    ctl = _CyclingCap([3, 7, 1, 12, 5])      # 12 is clamped to the block's 7 drafts
    res = dflash_generate(target, tok, d, prompt_ids=prompt, max_new_tokens=30, cap_controller=ctl)
    check_greedy_stream(tiny, prompt, res.token_ids, MIN_MATCH)
    assert len(ctl.updates) == res.num_rounds
    want = [min(c, 7) for c in (ctl.caps * res.num_rounds)[: res.num_rounds]]
    assert [dr for _, dr in ctl.updates] == want
    assert all(0 <= n <= dr for n, dr in ctl.updates)
    assert [n + 1 for n, _ in ctl.updates][:-1] == res.accept_lengths[:-1]


def test_dflash_generate_sampled_is_seeded(dev, tiny):
    from mlx_dspark import synthetic
    from mlx_dspark.generate import dflash_generate
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    d, cfg = synthetic.build_dflash(tiny.args, seed=9, num_hidden_layers=1, block_size=4, n_taps=2)
    d.bind(tiny)
    tok = SyntheticTokenizer(tiny.args.vocab_size)
    target = Target(tiny, tok)
    kw = dict(prompt_ids=list(range(20)), max_new_tokens=16, temperature=0.8, top_p=0.9, seed=123)
    a = dflash_generate(target, tok, d, **kw)
    b = dflash_generate(target, tok, d, **kw)
    c = dflash_generate(target, tok, d, **{**kw, "seed": 124})
    assert a.token_ids == b.token_ids
    assert a.token_ids != c.token_ids
    # sampled rounds replayed from one captured graph (Philox offset read from a device word)
    # draw exactly what the eager rounds draw
    e = dflash_generate(target, tok, d, use_graph=False, **kw)
    assert a.token_ids == e.token_ids and a.num_rounds >= 3


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_dflash_pipelined_rounds_match_sequential(dev, tiny, temperature):
    """Rounds enqueued one ahead of the host (two alternating round objects chained on the
    device) return the sequential rounds' ids, and cancelling the round enqueued past the last
    one leaves both caches (host and device lengths) where the sequential rounds leave them."""
    from mlx_dspark import synthetic
    from mlx_dspark.generate import _DFlashPipe, _DFlashRound, _pick
    from mlx_dspark.target import Target
    from mlx_dspark.tokenizer import SyntheticTokenizer
    print(f"pipelined DFlash rounds T={temperature}", flush=True)
    d, cfg = synthetic.build_dflash(tiny.args, seed=9, num_hidden_layers=2, block_size=8, n_taps=2)
    d.bind(tiny)
    target = Target(tiny, SyntheticTokenizer(tiny.args.vocab_size))
    prompt = np.random.default_rng(5).integers(0, tiny.args.vocab_size, 37).tolist()
    tap, cap, n_rounds = list(cfg.target_layer_ids), 7, 6

    def fresh():
        cache, dcache = target.make_cache(max_ctx=256), d.make_cache(max_ctx=256)
        logits, fused = tiny.prefill(prompt, cache, tap)
        d.ingest(fused, dcache)
        return cache, dcache, _pick(logits[0, -1], 0.0)

    cache, dcache, pending = fresh()
    rnd = _DFlashRound(target, d, cache, dcache, cap, temperature, 0.9, 0, 77)
    rnd.pending.fill_(pending)
    seq = [rnd.run(r, True) for r in range(n_rounds)]
    seq_lens = (list(cache.lengths), list(dcache.lengths))

    cache2, dcache2, pending2 = fresh()
    assert pending2 == pending
    pipe = _DFlashPipe(target, d, cache2, dcache2, cap, temperature, 0.9, 0, 77)
    pipe.start(pending2)
    pipe.enqueue()
    got = []
    for r in range(n_rounds):
        pipe.enqueue()                                   # the last one is past the end
        got.append(pipe.collect())
    pipe.cancel()
    torch.cuda.synchronize()
    assert got == seq
    assert (list(cache2.lengths), list(dcache2.lengths)) == seq_lens
    assert cache2.seq_lens.tolist() == cache.seq_lens.tolist() == seq_lens[0]
    assert dcache2.seq_lens.tolist() == dcache.seq_lens.tolist() == seq_lens[1]


def test_weight_prefetch_side_stream_leaves_the_forward_unchanged(dev, tiny):
    """prefetch_weights: each layer's o and gate|up weights read on a side stream during its
    attention stage; the logits and taps are bit-identical, eager and graph-replayed, and the
    cache lengths advance as without it."""
    print("weight prefetch on a side stream: tiny model, 8-bit KV, 64-token context, 16 rows", flush=True)
    model = tiny
    ctx = torch.randint(0, model.args.vocab_size, (1, 64), dtype=torch.int32, device=dev)
    ids = torch.randint(0, model.args.vocab_size, (1, 16), dtype=torch.int32, device=dev)
    outs = []
    for on in (False, True):
        model.prefetch_weights(on)
        cache = model.make_cache(max_ctx=128, kv_bits=8)
        model.forward(ctx, cache, None)
        eager = model.forward(ids, cache, [0, 1], advance=False)
        lo = torch.empty((16, model.args.vocab_size), dtype=torch.float32, device=dev)
        model.forward(ids, cache, [0, 1], advance=False, logits_out=lo)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            model.forward(ids, cache, [0, 1], advance=False, logits_out=lo)
        lo.zero_()
        g.replay()
        torch.cuda.synchronize()
        outs.append((eager[0].clone(), eager[1].clone(), lo.clone(), cache.lengths[0], int(cache.seq_lens[0])))
        del g
    model.prefetch_weights(False)
    (l0, f0, g0, n0, d0), (l1, f1, g1, n1, d1) = outs
    assert torch.equal(l0, l1) and torch.equal(f0, f1) and torch.equal(g0, g1)
    assert torch.equal(g0.view_as(l0), l0)
    assert (n0, d0) == (n1, d1) == (64, 64)


@pytest.mark.parametrize("nbytes", [16, 4080, 32768 + 16, (1 << 20) + 48])
def test_plain_read_kernel_ragged_sizes(dev, nbytes):
    """dsk_prefetch over sizes that end mid-chunk, from one workgroup to more workgroups than
    chunks: every load stays inside [p, p + bytes) (the lanes past the end re-read the last
    16 bytes), and the 16-byte sink is untouched for a buffer whose xor is not the sentinel."""
    from mlx_dspark import _hip
    from mlx_dspark._hip import ptr, stream_ptr
    print(f"plain read: {nbytes} bytes", flush=True)
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(16, dtype=torch.uint8, device=dev)
    for wg in (1, 3, 512, 4096):
        _hip.call("dsk_prefetch", ptr(buf), nbytes, wg, ptr(sink), stream_ptr())
    torch.cuda.synchronize()
    assert int(sink.sum()) == 0
