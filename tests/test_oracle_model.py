"""CPU pins for the model oracle: the reference's exact causal-mask grids, GQA attention
equal to explicitly tiled K/V, RoPE invariants, RMSNorm closed form, rollback semantics."""

import math

import numpy as np
import torch

from oracle import model as OM


def test_causal_mask_grids_match_reference():
    # tests/test_batch_engine.py:87-103 in the reference: offsets [2, 0], T=2 and [5, 3, 0], T=1
    assert OM.causal_mask(2, 2).int().tolist() == [[1, 1, 1, 0], [1, 1, 1, 1]]
    assert OM.causal_mask(0, 2).int().tolist() == [[1, 0], [1, 1]]
    assert OM.causal_mask(5, 1).int().tolist() == [[1, 1, 1, 1, 1, 1]]
    assert OM.causal_mask(3, 1).int().tolist() == [[1, 1, 1, 1]]
    assert OM.causal_mask(0, 1).int().tolist() == [[1]]


def test_gqa_attention_equals_tiled_kv():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(3, 8, 16, generator=g)
    K = torch.randn(5, 2, 16, generator=g)
    V = torch.randn(5, 2, 16, generator=g)
    got = OM.sdpa(q, K, V, 16 ** -0.5)
    Kt = K.repeat_interleave(4, dim=1)
    Vt = V.repeat_interleave(4, dim=1)
    s = torch.einsum("qhd,khd->hqk", q, Kt) * 16 ** -0.5
    ref = torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), Vt)
    assert torch.allclose(got, ref, atol=1e-5)


def test_rope_invariants():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 6, 128, generator=g, dtype=torch.float64).float()
    pos = torch.arange(6)
    r = OM.rope(x, pos, 1e6)
    assert torch.allclose(r.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)           # rotation
    assert torch.allclose(OM.rope(x, torch.zeros(6, dtype=torch.long), 1e6), x)  # position 0
    q = torch.randn(128, generator=g)
    k = torch.randn(128, generator=g)
    d1 = OM.rope(q[None, None], torch.tensor([7]), 1e4)[0, 0] @ OM.rope(k[None, None], torch.tensor([3]), 1e4)[0, 0]
    d2 = OM.rope(q[None, None], torch.tensor([14]), 1e4)[0, 0] @ OM.rope(k[None, None], torch.tensor([10]), 1e4)[0, 0]
    assert abs(float(d1 - d2)) < 1e-3                                          # relative position
    # closed form of one pair: dims (0, 64) rotate by pos * theta^0
    e = torch.zeros(1, 1, 128)
    e[0, 0, 0] = 1.0
    out = OM.rope(e, torch.tensor([2]), 1e6)[0, 0]
    assert abs(float(out[0]) - math.cos(2)) < 1e-6 and abs(float(out[64]) - math.sin(2)) < 1e-6


def test_rmsnorm_closed_form():
    x = torch.tensor([[3.0, 4.0]])
    w = torch.tensor([1.0, 2.0])
    out = OM.rmsnorm(x, w, 0.0)
    r = math.sqrt((9 + 16) / 2)
    assert torch.allclose(out, torch.tensor([[3 / r, 8 / r]]))


def test_normalized_metric_is_scale_invariant():
    a = torch.randn(2, 50)
    assert OM.normalized_maxdiff(a, 3.0 * a) < 1e-5


def test_gelu_tanh_matches_library():
    x = torch.linspace(-6, 6, 1001)
    ref = torch.nn.functional.gelu(x, approximate="tanh")
    assert torch.allclose(OM.gelu_tanh(x), ref, atol=1e-6)


def test_sliding_window_mask_bruteforce():
    off, W, win = 7, 4, 3
    m = OM.causal_mask(off, W, win)
    for i in range(W):
        for j in range(off + W):
            want = (j <= off + i) and (j > off + i - win)
            assert bool(m[i, j]) == want
    assert torch.equal(OM.causal_mask(off, W, 0), OM.causal_mask(off, W))
