"""GPU parity: greedy and sampled acceptance are bit-identical to the oracle (decisions,
sampled indices, rollback lengths), including the full [4, 17, 151936] acceptance config."""

import numpy as np
import pytest
import torch

from oracle import accept as A

pytestmark = pytest.mark.gpu


def _t(x, dev, dt=None):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev) if dt is None else torch.from_numpy(np.ascontiguousarray(x)).to(dev, dt)


@pytest.mark.parametrize("B,W,V,dtype", [(1, 16, 151936, "f32"), (2, 5, 1000, "f32"), (4, 9, 4099, "bf16"),
                                         (3, 1, 77, "f32")])
def test_accept_greedy_matches_oracle(dev, B, W, V, dtype):
    from mlx_dspark.ops import accept_greedy
    rng = np.random.default_rng(B * 100 + W)
    logits = rng.integers(-3, 4, size=(B, W, V)).astype(np.float32)   # plenty of exact ties
    tt_ref = logits.argmax(axis=2)
    draft = tt_ref[:, : W - 1].copy().astype(np.int32)
    for b in range(B):                                                  # break the match somewhere
        k = rng.integers(0, W)
        if k < W - 1:
            draft[b, k] = (draft[b, k] + 1) % V
    sl = rng.integers(0, 1000, size=B).astype(np.int32)
    if dtype == "bf16":
        lt = torch.from_numpy(logits).to(torch.bfloat16)
        ref = A.accept_greedy(lt.view(torch.int16).numpy().view(np.uint16), draft, sl, bf16_bits_in=True)
        lt = lt.to(dev)
    else:
        ref = A.accept_greedy(logits, draft, sl)
        lt = _t(logits, dev)
    sl_d = _t(sl, dev)
    tt, n, tok = accept_greedy(lt, _t(draft, dev) if W > 1 else None, seq_lens=sl_d)
    torch.cuda.synchronize()
    assert np.array_equal(tt.cpu().numpy(), ref["tt"])
    assert np.array_equal(n.cpu().numpy(), ref["n"])
    assert np.array_equal(tok.cpu().numpy(), ref["token"])
    assert np.array_equal(sl_d.cpu().numpy(), ref["seq_lens"])


CASES = [
    (2, 4, 1000, 1.0, 1.0, 0, False, False),
    (2, 4, 1000, 0.7, 0.9, 0, False, False),
    (2, 4, 1000, 1.0, 1.0, 50, True, False),
    (3, 3, 2048, 1.3, 0.8, 20, False, False),
    (2, 5, 999, 1.0, 0.95, 0, False, True),      # one-hot q (lookup drafts)
    (1, 2, 64, 0.5, 0.0, 0, False, False),       # empty nucleus
    (2, 3, 151936, 1.0, 0.95, 50, False, False), # both truncations at the vocabulary width
    (1, 0, 4096, 1.0, 0.9, 0, False, False),     # no drafts: only the bonus draw
    (2, 4, 3001, 0.8, 1e-6, 1, False, True),     # a one-element nucleus, top-1
    (2, 4, 151936, 0.6, 0.95, 20, True, False),  # a sampled round's settings at the vocabulary width
]


@pytest.mark.parametrize("B,L,V,T,tp,tk,mulinv,onehot", CASES)
def test_accept_sample_matches_oracle(dev, B, L, V, T, tp, tk, mulinv, onehot):
    from mlx_dspark.ops import accept_sample
    rng = np.random.default_rng(L * 31 + V)
    q = (rng.standard_normal((B, L, V)) * 3).astype(np.float32)
    p = np.concatenate([q + rng.standard_normal((B, L, V)).astype(np.float32),
                        rng.standard_normal((B, 1, V)).astype(np.float32) * 3], axis=1)
    # drafts: mostly the draft argmax (often accepted), some random
    draft = q.argmax(axis=2).astype(np.int32)
    if L:
        draft[:, -1] = rng.integers(0, V, size=B)
    sl = rng.integers(0, 500, size=B).astype(np.int32)
    for seed, off in [(1, 0), (2**40 + 7, 123456)]:
        ref = A.accept_sample(p, None if onehot else q, draft, T, tp, tk, mulinv, seed, off, sl)
        sl_d = _t(sl, dev)
        acc = torch.zeros((B, L), dtype=torch.uint8, device=dev)
        smp = torch.zeros((B, L + 1), dtype=torch.int32, device=dev)
        n, tok = accept_sample(_t(p, dev), None if onehot else _t(q, dev), _t(draft, dev), T, tp, tk,
                               q_mul_inv_t=mulinv, seed=seed, offset=off, seq_lens=sl_d, accept_out=acc,
                               sample_out=smp)
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), ref["accept"])
        assert np.array_equal(smp.cpu().numpy(), ref["sample"])
        assert np.array_equal(n.cpu().numpy(), ref["n"])
        assert np.array_equal(tok.cpu().numpy(), ref["token"])
        assert np.array_equal(sl_d.cpu().numpy(), ref["seq_lens"])


def test_accept_sample_full_acceptance_config(dev):
    """[4, 17, 151936] fp32: draft ~ N(0, 3^2), target = draft + N(0, 1), T=1, top_p=0.95."""
    from mlx_dspark.ops import accept_sample
    B, L, V = 4, 16, 151936
    g = torch.Generator().manual_seed(2024)
    q = torch.randn(B, L + 1, V, generator=g) * 3.0
    p = q + torch.randn(B, L + 1, V, generator=g)
    qn, pn = q[:, :L].contiguous().numpy(), p.numpy()
    draft = qn.argmax(axis=2).astype(np.int32)
    ref = A.accept_sample(pn, qn, draft, 1.0, 0.95, 0, False, 7, 11, np.zeros(B, np.int32))
    acc = torch.zeros((B, L), dtype=torch.uint8, device=dev)
    smp = torch.zeros((B, L + 1), dtype=torch.int32, device=dev)
    sl = torch.zeros(B, dtype=torch.int32, device=dev)
    n, tok = accept_sample(p.to(dev), q[:, :L].to(dev), _t(draft, dev), 1.0, 0.95, 0, seed=7, offset=11,
                           seq_lens=sl, accept_out=acc, sample_out=smp)
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy(), ref["accept"])
    assert np.array_equal(smp.cpu().numpy(), ref["sample"])
    assert np.array_equal(n.cpu().numpy(), ref["n"])
    assert np.array_equal(tok.cpu().numpy(), ref["token"])
    assert np.array_equal(sl.cpu().numpy(), ref["seq_lens"])


@pytest.mark.parametrize("T,tp,tk,mulinv", [(0.0, 1.0, 0, False), (1.0, 1.0, 0, False), (0.7, 0.9, 40, True)])
def test_sample_rows_matches_oracle(dev, T, tp, tk, mulinv):
    from mlx_dspark.ops import sample_rows
    rng = np.random.default_rng(5)
    R, V = 6, 5000
    logits = (rng.standard_normal((R, V)) * 2).astype(np.float32)
    ref_tok, ref_p = A.sample_rows(logits, T, tp, tk, mulinv, seed=99, offset=3, row0=4)
    pr = torch.full((R, V), -1.0, dtype=torch.float32, device=dev)
    tok, _ = sample_rows(_t(logits, dev), T, tp, tk, mul_inv_t=mulinv, seed=99, offset=3, row0=4, probs_out=pr)
    torch.cuda.synchronize()
    assert np.array_equal(tok.cpu().numpy(), ref_tok)
    if T > 0:
        assert np.array_equal(pr.cpu().numpy(), ref_p)


@pytest.mark.parametrize("R,V,ld,dtype", [(15, 151936, 151936, "f32"), (3, 77, 77, "f32"), (4, 4099, 4099, "bf16"),
                                         (5, 1000, 1003, "f32"), (2, 5000, 5008, "bf16"), (1, 8, 8, "f32")])
def test_argmax_rows_first_index_on_ties(dev, R, V, ld, dtype):
    """argmax_rows == numpy's argmax (first maximal index) on rows full of exact ties, aligned and
    unaligned row strides, f32 and bf16, a row of -inf; twice in a row on one workspace (the
    arrival counters must return to zero)."""
    from mlx_dspark.ops import argmax_rows, sample_rows
    print(f"argmax R={R} V={V} ld={ld} {dtype}", flush=True)
    rng = np.random.default_rng(R * 7 + V)
    for rep in range(2):
        full = rng.integers(-3, 4, size=(R, ld)).astype(np.float32)
        if R > 2:
            full[1, :V] = -np.inf
        ref = full[:, :V].argmax(axis=1).astype(np.int32)
        t = torch.from_numpy(full)
        if dtype == "bf16":
            t = t.to(torch.bfloat16)
        t = t.to(dev)[:, :V]
        tok = argmax_rows(t)
        tok2, _ = sample_rows(t.float() if dtype == "f32" else t, 0.0)
        torch.cuda.synchronize()
        assert np.array_equal(tok.cpu().numpy(), ref), rep
        assert np.array_equal(tok2.cpu().numpy(), ref), rep


@pytest.mark.parametrize("kind", ["equal", "ties", "spike", "tail"])
def test_accept_sample_degenerate_rows(dev, kind):
    """Rows whose threshold bucket holds the whole vocabulary (all-equal logits), rows of heavy
    exact ties, rows where one logit carries almost all the mass, and rows whose long flat tail
    of tiny probabilities (e ~ e^-12 each) holds about half the mass: the candidate select sees
    its largest and smallest inputs."""
    from mlx_dspark.ops import accept_sample
    B, L, V = 2, 3, 151936
    rng = np.random.default_rng({"equal": 1, "ties": 2, "spike": 3, "tail": 4}[kind])
    if kind == "equal":
        q = np.zeros((B, L, V), np.float32)
        p = np.zeros((B, L + 1, V), np.float32)
    elif kind == "ties":
        q = rng.integers(-3, 4, size=(B, L, V)).astype(np.float32)
        p = rng.integers(-3, 4, size=(B, L + 1, V)).astype(np.float32)
    elif kind == "spike":
        q = (rng.standard_normal((B, L, V))).astype(np.float32)
        p = (rng.standard_normal((B, L + 1, V))).astype(np.float32)
        p[:, :, 17] = 40.0
        q[:, :, 17] = 38.0
    else:   # one token at 12 over a tail near 0: each tail e ~ e^-12 < 2^-16, ~half the mass
        q = (0.01 * rng.standard_normal((B, L, V))).astype(np.float32)
        p = (0.01 * rng.standard_normal((B, L + 1, V))).astype(np.float32)
        p[:, :, 17] = 12.0
        q[:, :, 17] = 11.5
    draft = rng.integers(0, V, size=(B, L)).astype(np.int32)
    draft[:, 0] = 17
    for T, tp, tk in [(1.0, 0.95, 0), (1.0, 0.9, 1000), (0.6, 1.0, 7)]:
        print(f"degenerate {kind} T={T} top_p={tp} top_k={tk}", flush=True)
        ref = A.accept_sample(p, q, draft, T, tp, tk, False, 5, 9, np.zeros(B, np.int32))
        acc = torch.zeros((B, L), dtype=torch.uint8, device=dev)
        smp = torch.zeros((B, L + 1), dtype=torch.int32, device=dev)
        n, tok = accept_sample(_t(p, dev), _t(q, dev), _t(draft, dev), T, tp, tk, seed=5, offset=9,
                               accept_out=acc, sample_out=smp)
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), ref["accept"])
        assert np.array_equal(smp.cpu().numpy(), ref["sample"])
        assert np.array_equal(n.cpu().numpy(), ref["n"]) and np.array_equal(tok.cpu().numpy(), ref["token"])


def test_sample_rows_draft_block_shape(dev):
    """The DFlash draft rows: 15 x 151936 at T=0.6 / top-p 0.95 / top-k 20, tokens and the
    truncated distributions bit-exact."""
    from mlx_dspark.ops import sample_rows
    R, V = 15, 151936
    g = torch.Generator().manual_seed(8)
    logits = torch.randn(R, V, generator=g) * 3.0
    ref_tok, ref_p = A.sample_rows(logits.numpy(), 0.6, 0.95, 20, False, seed=3, offset=41, row0=0)
    pr = torch.empty((R, V), dtype=torch.float32, device=dev)
    tok, _ = sample_rows(logits.to(dev), 0.6, 0.95, 20, seed=3, offset=41, probs_out=pr)
    torch.cuda.synchronize()
    assert np.array_equal(tok.cpu().numpy(), ref_tok)
    assert np.array_equal(pr.cpu().numpy(), ref_p)


def test_offset_word_on_device_equals_host_offset(dev):
    """offset_dev holding k draws exactly what offset=k draws (sample_rows and accept_sample),
    and rounds k and k + 1 draw different uniforms."""
    from mlx_dspark.ops import accept_sample, sample_rows
    R, V, L = 8, 4096, 6
    rng = np.random.default_rng(12)
    logits = torch.from_numpy((rng.standard_normal((R, V)) * 2).astype(np.float32)).to(dev)
    p = torch.from_numpy((rng.standard_normal((1, L + 1, V)) * 2).astype(np.float32)).to(dev)
    q = torch.from_numpy((rng.standard_normal((1, L, V)) * 2).astype(np.float32)).to(dev)
    draft = torch.from_numpy(rng.integers(0, V, size=(1, L)).astype(np.int32)).to(dev)
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    outs = []
    for k in (5, 6):
        word.fill_(k)
        t_host, _ = sample_rows(logits, 1.0, 0.9, 0, seed=21, offset=k)
        t_dev, _ = sample_rows(logits, 1.0, 0.9, 0, seed=21, offset=999, offset_dev=word)
        smp_h = torch.zeros((1, L + 1), dtype=torch.int32, device=dev)
        smp_d = torch.zeros((1, L + 1), dtype=torch.int32, device=dev)
        acc_h = torch.zeros((1, L), dtype=torch.uint8, device=dev)
        acc_d = torch.zeros((1, L), dtype=torch.uint8, device=dev)
        accept_sample(p, q, draft, 1.0, 0.9, 0, seed=21, offset=k, accept_out=acc_h, sample_out=smp_h)
        accept_sample(p, q, draft, 1.0, 0.9, 0, seed=21, offset=999, offset_dev=word, accept_out=acc_d,
                      sample_out=smp_d)
        torch.cuda.synchronize()
        assert torch.equal(t_host, t_dev) and torch.equal(smp_h, smp_d) and torch.equal(acc_h, acc_d)
        ref = A.sample_rows(logits.cpu().numpy(), 1.0, 0.9, 0, False, seed=21, offset=k)[0]
        assert np.array_equal(t_host.cpu().numpy(), ref)
        outs.append((t_host.cpu(), smp_h.cpu()))
    assert not torch.equal(outs[0][0], outs[1][0]) or not torch.equal(outs[0][1], outs[1][1])
