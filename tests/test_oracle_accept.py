"""CPU checks that pin the acceptance oracle (oracle/accept_oracle.c) to things other than
itself: published Philox vectors, libm, the reference's float64 sort+cumsum truncation, exact
rational arithmetic for the top-p target, the exact output distribution of speculative
sampling, and brute force for greedy accept and for the GPU's order-free threshold rule."""

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import accept as A


def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds
    assert [int(x) for x in A.philox([0, 0, 0, 0], [0, 0])] == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert [int(x) for x in A.philox([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2)] == [
        0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert [int(x) for x in A.philox([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344],
                                     [0xA4093822, 0x299F31D0])] == [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def _ulp_err(got: float, want: float) -> float:
    g = np.float32(got)
    w = np.float32(want)
    return abs(float(g) - float(want)) / float(np.spacing(w))


def test_expf_matches_libm_within_2ulp():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-86.0, 0.0, 20000), rng.uniform(-1, 1, 5000), [0.0, -1e-8, -85.99, 1.0, 10.0, 88.0]])
    worst = 0.0
    for x in xs.astype(np.float32):
        worst = max(worst, _ulp_err(A.expf(float(x)), math.exp(float(x))))
    assert worst <= 2.0, worst
    assert A.expf(-86.5) == 0.0 and A.expf(-1000.0) == 0.0
    assert A.expf(0.0) == 1.0


@pytest.mark.parametrize("T,top_p,top_k", [(1.0, 1.0, 0), (1.0, 0.95, 0), (0.7, 1.0, 50), (1.0, 0.9, 20),
                                           (1.3, 0.5, 0), (0.5, 0.99, 1000)])
def test_probs_match_reference_sort_cumsum(T, top_p, top_k):
    rng = np.random.default_rng(1)
    for trial in range(5):
        V = int(rng.integers(50, 3000))
        logits = (rng.standard_normal(V) * 3.0).astype(np.float32)
        got = A.probs(logits, T, top_p, top_k).astype(np.float64)
        ref = A.truncate_probs_ref(A.softmax64(logits.astype(np.float64) / T), top_p, top_k)
        # same support (no near-ties at the boundary for continuous random logits) ...
        assert np.array_equal(got > 0, ref > 0), (trial, V)
        # ... and the same values to float32 accuracy
        assert np.max(np.abs(got - ref)) < 2e-6


def test_probs_identity_path_is_plain_softmax():
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -2.0], np.float32)
    got = A.probs(x, 1.0, 1.0, 0)
    assert np.allclose(got, A.softmax64(x), atol=1e-7)


def test_probs_ties_at_boundary_are_kept():
    # four equal logits at the top: top_k=2 keeps all four ties (p >= kth), as the reference does
    x = np.array([5, 5, 5, 5, 0, 0, -1], np.float32)
    p = A.probs(x, 1.0, 1.0, 2)
    assert np.count_nonzero(p) == 4
    # nucleus: with top_p just above one tie's mass, all tied values survive
    p2 = A.probs(x, 1.0, 0.26, 0)
    assert np.count_nonzero(p2) == 4


def test_top_p_zero_gives_empty_distribution():
    x = np.array([3, 1, 0], np.float32)
    assert np.all(A.probs(x, 1.0, 0.0, 0) == 0)


def _exact_output_distribution(p, q):
    """P(out = x) for one draft position: accept q-sample with prob min(1, p/q), else residual."""
    acc = np.minimum(q, p)                     # q(x) * min(1, p(x)/q(x))
    resid = np.maximum(p - q, 0)
    rej = 1.0 - acc.sum()
    r = resid / resid.sum() if resid.sum() > 0 else resid
    return acc + rej * r


@pytest.mark.parametrize("T,tp,tk", [(1.0, 1.0, 0), (1.0, 0.8, 0), (0.7, 1.0, 3)])
def test_speculative_sampling_is_lossless_exactly(T, tp, tk):
    target = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -2.0], np.float32)
    draft = target[::-1].copy()
    p = A.probs(target, T, tp, tk).astype(np.float64)
    q = A.probs(draft, T, tp, tk).astype(np.float64)
    out = _exact_output_distribution(p, q)
    ref = A.truncate_probs_ref(A.softmax64(target.astype(np.float64) / T), tp, tk)
    assert np.max(np.abs(out - ref)) < 1e-6


@pytest.mark.parametrize("T,tp,tk", [(1.0, 1.0, 0), (1.0, 0.8, 0), (0.7, 1.0, 3)])
def test_statistical_kat_losslessness(T, tp, tk):
    # replay of the reference's test_topp_speculative_sampling_is_lossless with Philox draws:
    # V=6, target logits [2,1,.5,0,-1,-2], draft logits reversed, 20000 rounds. The engine
    # derives q from draft logits with the same temperature and truncation as p (what the
    # reference's drafters pass in), so the proposal is drawn from that same q.
    V = 6
    target = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -2.0], np.float32)
    qlog = target[::-1].copy()
    vlog = np.stack([target, target])[None]            # [1, 2, V]
    qtrunc = A.probs(qlog, T, tp, tk)
    counts = np.zeros(V)
    for r in range(20000):
        x = A.categorical(qtrunc, int(A.philox([r, 0, 7, 0], [1, 2])[0]))
        res = A.accept_sample(vlog, qlog[None, None], np.array([[x]]), T, tp, tk, seed=12345, offset=r)
        counts[x if res["n"][0] == 1 else res["token"][0]] += 1
    emp = counts / counts.sum()
    exp = A.truncate_probs_ref(A.softmax64(target.astype(np.float64) / T), tp, tk)
    assert np.abs(emp - exp).max() < 0.02, (emp, exp)


def test_categorical_inverse_cdf():
    w = np.array([0.0, 0.25, 0.0, 0.75], np.float32)
    assert A.categorical(w, 0) == 1                              # u = 0 -> first positive mass
    assert A.categorical(w, 0xFFFFFFFF) == 3                     # u -> 1 -> last positive mass
    assert A.categorical(w, int(0.25 * 2**32) - 256) == 1
    assert A.categorical(w, int(0.25 * 2**32)) == 3
    assert A.categorical(np.zeros(8, np.float32), 0x80000000) == 4   # all-zero: uniform index


def test_greedy_accept_bruteforce():
    rng = np.random.default_rng(3)
    V, W = 5, 4
    for _ in range(300):
        logits = rng.integers(0, 3, size=(2, W, V)).astype(np.float32)   # many ties
        draft = rng.integers(0, V, size=(2, W - 1)).astype(np.int32)
        res = A.accept_greedy(logits, draft, seq_lens=np.array([10, 20], np.int32))
        for b in range(2):
            tt = [int(np.flatnonzero(logits[b, i] == logits[b, i].max())[0]) for i in range(W)]
            n = 0
            while n < W - 1 and draft[b, n] == tt[n]:
                n += 1
            assert list(res["tt"][b]) == tt
            assert res["n"][b] == n and res["token"][b] == tt[n]
            assert res["seq_lens"][b] == [10, 20][b] + n + 1


def test_accept_sample_all_accept_takes_bonus_from_last_row():
    # identical p and q rows: min(1, p/q) = 1, every draft accepted, the token is a bonus draw
    rng = np.random.default_rng(4)
    V, L = 50, 3
    p = rng.standard_normal((1, L + 1, V)).astype(np.float32)
    draft = np.array([[1, 2, 3]], np.int32)
    res = A.accept_sample(p, p[:, :L], draft, 1.0, seed=9)
    assert res["n"][0] == L
    assert res["token"][0] == res["sample"][0, L]


def test_top_p_target_is_the_exact_ceiling():
    rng = np.random.default_rng(5)
    for _ in range(3000):
        top_p = np.float32(rng.uniform(0.0, 1.0))
        Z = int(rng.integers(2**31, 2**50))
        assert A.top_p_target(top_p, Z) == math.ceil(Fraction(float(top_p)) * Z)
    assert A.top_p_target(0.0, 2**50) == 0 and A.top_p_target(-0.5, 2**50) == 0
    assert A.top_p_target(1e-40, 2**31) == 1                       # subnormal top_p: keeps the top
    assert A.top_p_target(0.5, 2**31 + 1) == 2**30 + 1              # ceiling, not floor
    top = float(np.nextafter(np.float32(1.0), np.float32(0.0)))
    Z = 2**50 + 12345
    assert A.top_p_target(top, Z) == math.ceil(Fraction(top) * Z)


def _fx(e):
    return np.floor(np.asarray(e, np.float64) * 2.0**31).astype(np.int64)


def _kept_by_max_rule(e, top_k, top_p):
    """The GPU's rule: both thresholds from the untruncated row, keep e >= the larger one."""
    V = e.size
    w = _fx(e)
    vals = np.sort(e)[::-1]
    kth = float(vals[top_k - 1]) if 0 < top_k < V else 0.0
    cut = 0.0
    if top_p < 1.0:
        TP = A.top_p_target(top_p, int(w.sum()))
        if TP == 0:
            return np.zeros(V, bool)
        cands = [float(c) for c in np.unique(e)[::-1] if int(w[e >= c].sum()) >= TP]
        cut = cands[0]
    return e >= max(kth, cut)


def test_order_free_threshold_rule_matches_sequential_truncation():
    rng = np.random.default_rng(6)
    checked = 0
    for _ in range(3000):
        V = int(rng.integers(2, 40))
        logits = rng.integers(-4, 5, size=V).astype(np.float32) * np.float32(rng.choice([0.5, 1.0, 3.0]))
        T = float(rng.choice([0.7, 1.0, 1.5]))
        top_k = int(rng.integers(0, V + 2))
        top_p = float(rng.choice([1.0, 0.0, rng.uniform(0.05, 1.0)]))
        y = logits / np.float32(T)
        e = np.array([A.expf(float(v - y.max())) for v in y], np.float32)
        got = A.probs(logits, T, top_p, top_k) > 0
        want = _kept_by_max_rule(e, top_k, top_p) & (e > 0)
        assert np.array_equal(got, want), (logits, T, top_k, top_p)
        checked += int(0 < top_k < V and top_p < 1.0)
    assert checked > 500                    # both truncations together, many times
