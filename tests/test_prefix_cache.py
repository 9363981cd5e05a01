"""CPU checks of the prefix KV cache (slot choice, trimming, LRU, store re-validation, spill
round trips), on paged caches allocated on the CPU. The reference's own behaviour it follows:
src/mlx_dspark/prefix_cache.py:128-161 (acquire / store)."""

import pytest
import torch

from mlx_dspark.kv import PagedKVCache
from mlx_dspark.prefix_cache import PrefixCache, _lcp, target_cache_reusable


def _mk(kv_bits=None, layers=2):
    return lambda: PagedKVCache(layers, 1, 2, 64, 256, page=16, kv_bits=kv_bits, device="cpu")


def _filled(make, n, seed):
    """A cache holding n positions of seeded random pool contents."""
    c = make()
    g = torch.Generator().manual_seed(seed)
    for pools in (c.k, c.v, c.k_sb, c.v_sb):
        for t in pools:
            if t is not None:
                t.copy_(torch.randint(0, 250, t.shape, generator=g).to(t.dtype))
    c.set_lengths([n])
    return c


def test_lcp():
    assert _lcp([], [1]) == 0
    assert _lcp([1, 2, 3], [1, 2, 3]) == 3
    assert _lcp([1, 2, 3], [1, 2, 4, 5]) == 2
    assert _lcp([7], [8]) == 0
    assert _lcp(list(range(100)), list(range(50))) == 50


def test_reuse_longest_prefix_and_checkout():
    make = _mk()
    pc = PrefixCache(make, min_reuse=4, slots=3)
    a = list(range(100, 140))
    b = list(range(200, 230))
    pc.store(_filled(make, 40 + 9, 1), None, a, list(range(10)))          # holds a + 9 generated
    pc.store(_filled(make, 30 + 4, 2), None, b, list(range(5)))
    assert [s["tokens"] for s in pc.info()["slots"]] == [34, 49]
    # the turn after `a`: its prompt extends a's record
    nxt = a + list(range(9)) + [77, 78]
    cache, ctx, reuse = pc.acquire(nxt)
    assert reuse == 49 and ctx is None and cache.lengths == [49] and int(cache.seq_lens[0]) == 49
    assert [s["tokens"] for s in pc.info()["slots"]] == [34]             # checked out
    assert pc.info()["hits"] == 1 and pc.info()["reused_tokens"] == 49
    # a prompt diverging early cuts the cache to the shared prefix
    pc.store(cache, None, nxt, [5, 6, 7])
    cache, _, reuse = pc.acquire(a[:20] + [1, 2, 3])
    assert reuse == 20 and cache.lengths == [20]


def test_reuse_leaves_one_prompt_token_and_respects_min_reuse():
    make = _mk()
    pc = PrefixCache(make, min_reuse=8)
    p = list(range(10, 30))
    pc.store(_filled(make, 25, 3), None, p, [1, 2, 3, 4, 5, 6])
    _, _, reuse = pc.acquire(p)                      # identical prompt: one token left to prefill
    assert reuse == len(p) - 1
    pc2 = PrefixCache(make, min_reuse=8)
    pc2.store(_filled(make, 25, 3), None, p, [1, 2, 3, 4, 5, 6])
    cache, _, reuse = pc2.acquire(p[:7] + [999])      # 7 shared < min_reuse: fresh caches
    assert reuse == 0 and cache.lengths == [0] and len(pc2.info()["slots"]) == 1


def test_lru_eviction_keeps_most_recent():
    make = _mk()
    pc = PrefixCache(make, min_reuse=2, slots=2)
    for i in range(3):
        p = [1000 * (i + 1) + j for j in range(10)]
        pc.store(_filled(make, 12, i), None, p, [1, 2, 3])
    assert len(pc.info()["slots"]) == 2
    _, _, reuse = pc.acquire([1000 + j for j in range(10)] + [5])    # the first one was evicted
    assert reuse == 0
    _, _, reuse = pc.acquire([3000 + j for j in range(10)] + [5])
    assert reuse == 10


def test_store_claims_only_what_the_caches_hold():
    make = _mk()
    pc = PrefixCache(make, min_reuse=1, make_ctx=_mk(layers=1))
    p = list(range(50))
    short = _filled(make, 45, 4)                     # fewer than prompt + 9 generated - 1
    ctx = _filled(_mk(layers=1), 52, 5)
    pc.store(short, ctx, p, list(range(10)))
    assert pc.info()["slots"][0]["tokens"] == 45 and ctx.lengths == [45]
    long = _filled(make, 70, 6)                      # a stale tail past the record is cut
    pc.store(long, None, p, [1, 2])
    assert pc.info()["slots"][0]["tokens"] == 51 and long.lengths == [51]


@pytest.mark.parametrize("kv_bits", [None, 8])
def test_spill_round_trip_is_bit_exact(tmp_path, kv_bits):
    make, make_ctx = _mk(kv_bits), _mk(kv_bits, layers=1)
    pc = PrefixCache(make, make_ctx, min_reuse=4, l2_dir=str(tmp_path), max_ram_bytes=1, slots=2)
    p = list(range(300, 340))
    cache, ctx = _filled(make, 45, 7), _filled(make_ctx, 45, 8)
    keep = {name: [t.clone() for t in pools if t is not None]
            for name, pools in (("k", cache.k), ("v", cache.v), ("k_sb", cache.k_sb), ("ctx_k", ctx.k))}
    pc.store(cache, ctx, p, list(range(6)))
    assert pc.info()["slots"][0]["spilled"] and len(list(tmp_path.iterdir())) == 2
    got, gctx, reuse = pc.acquire(p + [5, 5])
    assert reuse == 40 and got is not cache and got.lengths == [40] and gctx.lengths == [40]
    # positions < reuse sit in the first pages of row 0 in both caches (identity block table)
    npg = (45 + 15) // 16
    for a, b in zip(keep["k"] + keep["v"], got.k + got.v):
        assert torch.equal(a[:npg], b[:npg])
    for a, b in zip(keep["k_sb"], [t for t in got.k_sb if t is not None]):
        assert torch.equal(a[:npg], b[:npg])
    assert torch.equal(keep["ctx_k"][0][:npg], gctx.k[0][:npg])
    pc.reset()
    assert list(tmp_path.iterdir()) == [] and pc.info()["slots"] == []


def test_paged_caches_are_always_reusable():
    assert target_cache_reusable(_mk()())
