"""CPU checks of the page-level prefix KV store on paged caches allocated on the CPU: which
prefix a prompt reuses (the reference's rule, src/mlx_dspark/prefix_cache.py:128-161: the
longest common prefix with a stored conversation, at least one prompt token left to
prefill, ``min_reuse``), that row 0 then reads exactly the stored K/V of those positions,
that conversations share whole pages and stores copy nothing, copy-on-write of the page a
reuse ends in, branch eviction, pins, and bit-exact spill round trips."""

import pytest
import torch

from mlx_dspark.kv import PagedKVCache
from mlx_dspark.prefix_cache import PrefixCache, _Arena, _lcp, target_cache_reusable

PAGE = 16


def _mk(kv_bits=None, layers=2, max_ctx=256):
    return lambda spare_rows=0: PagedKVCache(layers, 1, 2, 64, max_ctx, page=PAGE, kv_bits=kv_bits, device="cpu",
                                             spare_rows=spare_rows)


def _val(tok, pos, layer, salt=0):
    return (tok * 7 + pos * 3 + layer * 5 + salt) % 251


def _write(cache, tokens, start, end, salt=0):
    """Position p of row 0 gets a value that names (tokens[p], p, layer) in every pool."""
    bt = cache.row_pages(0)
    for p in range(start, end):
        pg, sl = bt[p // cache.page], p % cache.page
        for l in range(cache.n_layers):
            v = _val(tokens[p], p, l, salt)
            cache.k[l][pg, :, sl, :] = v
            cache.v[l][pg, :, sl, :] = v + 1
            if cache.k_sb[l] is not None:
                cache.k_sb[l][pg, :, sl, :] = 1000 * v + 3
                cache.v_sb[l][pg, :, sl, :] = 1000 * v + 4


def _check(cache, tokens, n, salt=0):
    bt = cache.row_pages(0)
    for p in range(n):
        pg, sl = bt[p // cache.page], p % cache.page
        for l in range(cache.n_layers):
            v = _val(tokens[p], p, l, salt)
            assert int(cache.k[l][pg, 0, sl, 0]) == v, (p, l)
            assert int(cache.v[l][pg, 1, sl, 63]) == v + 1, (p, l)
            if cache.k_sb[l] is not None:
                assert int(cache.k_sb[l][pg, 1, sl, 0]) == 1000 * v + 3


def _serve(pc, prompt, gen, held=None, ctx_held=None, salt=0):
    """The server's acquire -> generate -> store flow with a generation that writes every
    position it feeds (prompt suffix and all generated tokens but the last) plus junk past it."""
    cache, ctx, reuse = pc.acquire(prompt)
    seq = list(prompt) + list(gen)
    n = len(seq) - 1 if held is None else held
    for c, h in ((cache, n), (ctx, n if ctx_held is None else ctx_held)):
        if c is None:
            continue
        assert c.lengths == [reuse]
        _check(c, seq, reuse, salt)                       # what it reuses is what was stored
        _write(c, seq, reuse, h, salt)
        junk = min(h + 5, c.max_ctx)
        _write(c, [999] * junk, h, junk, salt=77)         # rejected drafts past the length
        c.set_lengths([h])
    pc.store(cache, ctx, prompt, gen)
    return reuse


def test_lcp():
    assert _lcp([], [1]) == 0
    assert _lcp([1, 2, 3], [1, 2, 3]) == 3
    assert _lcp([1, 2, 3], [1, 2, 4, 5]) == 2
    assert _lcp([7], [8]) == 0
    assert _lcp(list(range(100)), list(range(50))) == 50


def test_turns_reuse_the_whole_conversation():
    pc = PrefixCache(_mk(), _mk(layers=1), min_reuse=4)
    t1 = list(range(100, 140))
    g1 = list(range(500, 510))
    assert _serve(pc, t1, g1) == 0
    t2 = t1 + g1 + [77, 78]
    assert _serve(pc, t2, [1, 2, 3]) == len(t1) + len(g1) - 1
    assert pc.info()["hits"] == 1 and pc.info()["reused_tokens"] == 49
    t3 = t2 + [1, 2] + [5]
    assert _serve(pc, t3, [9]) == len(t2) + 2
    info = pc.info()
    assert len(info["slots"]) == 1 and info["slots"][0]["tokens"] == len(t3)   # one branch


def test_conversations_share_whole_pages():
    pc = PrefixCache(_mk(), min_reuse=4, slots=4)
    system = list(range(1000, 1040))                      # 2.5 pages
    a, b = system + list(range(10, 30)), system + list(range(40, 70))
    _serve(pc, a, [1, 2, 3])
    stored_a = pc.info()["pages"]["stored"]
    assert _serve(pc, b, [4, 5]) == 40                    # reuse ends inside page 2: copy on write
    info = pc.info()
    # b's pages 0 and 1 are a's pages; b adds its own pages from page 2 on
    assert info["pages"]["stored"] == stored_a + (-(-(len(b) + 1) // PAGE) - 2)
    assert info["pages"]["shared"] == 1 and len(info["slots"]) == 2
    for prompt, gen in ((a, [1, 2, 3]), (b, [4, 5])):     # both conversations intact
        q = prompt + gen[:-1] + [0]
        cache, _, reuse = pc.acquire(q)
        assert reuse == len(prompt) + len(gen) - 1
        _check(cache, prompt + gen, reuse)
        pc.store(cache, None, q, [0])


def test_store_copies_nothing_and_a_mid_page_reuse_copies_one_page(monkeypatch):
    copies = []
    orig = _Arena.copy_page
    monkeypatch.setattr(_Arena, "copy_page", lambda self, s, d: (copies.append((s, d)), orig(self, s, d)))
    pc = PrefixCache(_mk(), _mk(layers=1), min_reuse=4)
    p = list(range(64))                                   # exactly 4 pages
    _serve(pc, p, [1])
    assert copies == []
    assert _serve(pc, p[:32] + [7, 7, 7], [2]) == 32      # page-aligned reuse: no copy
    assert copies == []
    assert _serve(pc, p[:40] + [8], [3]) == 40            # ends inside page 2: one page per arena
    assert len(copies) == 2


def test_copy_on_write_keeps_the_stored_page():
    pc = PrefixCache(_mk(), min_reuse=4, slots=3)
    a = list(range(200, 236))
    _serve(pc, a, [1, 2])
    b = a[:20] + list(range(300, 330))                    # shares 20 tokens: inside page 1
    assert _serve(pc, b, [3]) == 20
    cache, _, reuse = pc.acquire(a + [1, 9])
    assert reuse == len(a) + 1
    _check(cache, a + [1, 2], reuse)                      # a's page 1 was not written by b
    pc.store(cache, None, a + [1, 9], [0])


def test_reuse_leaves_one_prompt_token_and_respects_min_reuse():
    pc = PrefixCache(_mk(), min_reuse=8)
    p = list(range(10, 30))
    _serve(pc, p, [1, 2, 3, 4, 5, 6])
    assert _serve(pc, p, [1]) == len(p) - 1               # identical prompt: one token to prefill
    assert _serve(pc, p[:7] + [999], [1]) == 0            # 7 shared < min_reuse


def test_lru_branch_eviction():
    pc = PrefixCache(_mk(), min_reuse=2, slots=2)
    prompts = [[1000 * (i + 1) + j for j in range(40)] for i in range(3)]
    for p in prompts:
        _serve(pc, p, [1, 2, 3])
    info = pc.info()
    assert len(info["slots"]) == 2
    assert info["pages"]["stored"] == 2 * -(-42 // PAGE)  # the oldest branch's pages went back
    assert _serve(pc, prompts[0] + [5], [1]) == 0
    assert _serve(pc, prompts[2] + [5], [1]) == 40        # the newest survived


def test_store_claims_only_what_the_caches_hold():
    pc = PrefixCache(_mk(), _mk(layers=1), min_reuse=1)
    p = list(range(50))
    _serve(pc, p, list(range(10)), held=45, ctx_held=52)
    assert pc.info()["slots"][0]["tokens"] == 45
    _serve(pc, p + [7], [1, 2], held=48, ctx_held=44)     # the shorter arena bounds the record
    assert pc.info()["slots"][0]["tokens"] in (44, 45)
    cache, ctx, reuse = pc.acquire(p + [7, 8])
    assert reuse == 45


def test_checkout_is_exclusive_and_reset_returns_everything(tmp_path):
    pc = PrefixCache(_mk(), min_reuse=2, l2_dir=str(tmp_path), max_ram_bytes=1)
    _serve(pc, list(range(40)), [1])
    cache, _, _ = pc.acquire(list(range(40)))
    with pytest.raises(RuntimeError):
        pc.acquire([1, 2, 3])
    with pytest.raises(ValueError):
        pc.store(PagedKVCache(2, 1, 2, 64, 64, page=PAGE, device="cpu"), None, [1], [2])
    pc.reset()
    assert pc.info()["slots"] == [] and list(tmp_path.iterdir()) == []
    assert all(len(a.free) == a.cache.n_pages for a in pc.arenas)
    assert pc.acquire([1, 2, 3])[2] == 0


def test_pinned_pages_survive_eviction_pressure():
    pc = PrefixCache(_mk(max_ctx=64), min_reuse=2, slots=1)   # 4 pages a row, 8 in the arena
    a = list(range(50))
    _serve(pc, a, [1])
    cache, _, reuse = pc.acquire(a[:48] + [3])            # pins a's first 3 pages
    assert reuse == 48
    _check(cache, a, 48)
    free = len(pc.arenas[0].free)
    assert free == 8 - 4 - 1                              # row 0 holds 4 pages, a's tail page is stored
    _write(cache, a[:48] + [3, 4], 48, 50)
    cache.set_lengths([50])
    pc.store(cache, None, a[:48] + [3], [4, 5])
    _check(pc.acquire(a[:48] + [3, 4, 9])[0], a[:48] + [3, 4], 50)


@pytest.mark.parametrize("kv_bits", [None, 8])
def test_spill_round_trip_is_bit_exact(tmp_path, kv_bits):
    pc = PrefixCache(_mk(kv_bits), _mk(kv_bits, layers=1), min_reuse=4, l2_dir=str(tmp_path), max_ram_bytes=1,
                     slots=2)
    p = list(range(300, 340))
    _serve(pc, p, list(range(6)))
    info = pc.info()
    assert info["slots"][0]["spilled"] and info["pages"]["resident"] == 0
    assert len(list(tmp_path.iterdir())) == info["pages"]["stored"] == 3
    cache, ctx, reuse = pc.acquire(p + [5, 5])
    assert reuse == 40 and cache.lengths == [40] and ctx.lengths == [40]
    _check(cache, p + list(range(6)), 40)
    _check(ctx, p + list(range(6)), 40)
    pc.store(cache, ctx, p + [5, 5], [1])
    pc.reset()
    assert list(tmp_path.iterdir()) == [] and pc.info()["slots"] == []


def test_spill_budget_keeps_the_newest_pages_resident(tmp_path):
    make = _mk()
    page_bytes = _Arena(make()).page_bytes
    pc = PrefixCache(make, min_reuse=2, l2_dir=str(tmp_path), max_ram_bytes=3 * page_bytes, slots=4)
    _serve(pc, list(range(100, 164)), [1])                # 4 pages
    _serve(pc, list(range(200, 264)), [1])                # 4 more: 5 spill, leaves first
    info = pc.info()
    assert info["pages"]["resident"] == 3 and info["pages"]["stored"] == 8
    assert _serve(pc, list(range(100, 164)) + [1, 2], [3]) == 64


def test_paged_caches_are_always_reusable():
    assert target_cache_reusable(_mk()())


def _free(pc):
    return [len(a.free) for a in pc.arenas]


def test_failed_acquire_returns_every_page_it_took():
    # the second arena's allocation fails after the first arena's private pages were taken and
    # set into row 0: they go back to the free list and row 0 is left empty in both arenas
    pc = PrefixCache(_mk(), _mk(layers=1), min_reuse=4)
    p = list(range(100, 140))
    _serve(pc, p, [1, 2, 3])
    before = _free(pc)
    real = pc._alloc

    def alloc(ai, n):
        if ai == 1:
            raise RuntimeError("planted: no pages in the second arena")
        return real(ai, n)

    pc._alloc = alloc
    with pytest.raises(RuntimeError, match="planted"):
        pc.acquire(p + [1, 2, 9])
    assert _free(pc) == before and [a.cache.lengths for a in pc.arenas] == [[0], [0]]
    assert pc._out is None
    pc._alloc = real
    assert _serve(pc, p + [1, 2, 9], [4]) == len(p) + 2          # the stored prefix is intact


def test_failed_load_of_a_spilled_page_returns_its_pages(tmp_path):
    # a spilled page whose file no longer matches the arena layout: the load fails after the
    # first arena's page was allocated for it; that page goes back and the node stays spilled
    pc = PrefixCache(_mk(), _mk(layers=1), min_reuse=4, l2_dir=str(tmp_path), max_ram_bytes=1, slots=2)
    p = list(range(300, 340))
    _serve(pc, p, list(range(6)))
    assert pc.info()["pages"]["resident"] == 0
    from safetensors.torch import load_file, save_file
    for f in tmp_path.iterdir():
        data = load_file(str(f))
        data = {k: (v[..., :1].contiguous() if k.startswith("1.") else v) for k, v in data.items()}
        save_file(data, str(f))
    before = _free(pc)
    with pytest.raises(ValueError, match="does not match the arena layout"):
        pc.acquire(p + [5, 5])
    assert _free(pc) == before and pc.info()["pages"]["resident"] == 0 and pc._out is None
