"""Prefix KV reuse across requests over paged caches (src/mlx_dspark/prefix_cache.py:111-249).

A small LRU of finished conversations. Each slot is a target PagedKVCache (plus, for DSpark,
the drafter's context cache) and the token record those caches hold. ``acquire(prompt)``
checks out the slot with the longest common prefix, trims its caches to that prefix and hands
them to the generation, which then prefills only the suffix. Trimming is length arithmetic on
the device ``seq_lens``: kept positions hold K already roped at their absolute position, and
sliding-window layers keep every key (the window is a mask in the attention kernel), so any
earlier position is a valid cut and no layer ever refuses reuse. ``store()`` re-validates a
finished generation's caches as the most recent slot.

Slots are whole caches in HBM; ``max_ram_bytes`` budgets their device bytes. Past the budget
the least recent slots spill to safetensors files under ``l2_dir`` (the used pages of every
layer, plus the token record) and reload into fresh caches on their next reuse.
"""

from __future__ import annotations

import glob
import json
import math
import os

import numpy as np
import torch

from .kv import PagedKVCache


def _lcp(a, b) -> int:
    """Length of the longest common prefix of two id sequences."""
    n = min(len(a), len(b))
    if n == 0:
        return 0
    x = np.asarray(a[:n], dtype=np.int64) != np.asarray(b[:n], dtype=np.int64)
    return int(np.argmax(x)) if x.any() else n


def target_cache_reusable(cache) -> bool:
    """True when every layer of ``cache`` can be cut back to any earlier position: always for a
    PagedKVCache; other cache objects need ``offset`` and ``trim``."""
    if isinstance(cache, PagedKVCache):
        return True
    return all(hasattr(c, "trim") and hasattr(c, "offset") for c in cache)


def _held(cache) -> int:
    return int(cache.lengths[0]) if isinstance(cache, PagedKVCache) else int(cache[0].offset)


def _cut(cache, n: int) -> None:
    if isinstance(cache, PagedKVCache):
        cache.trim_to(n)
    else:
        for c in cache:
            extra = int(c.offset) - n
            if extra > 0:
                c.trim(extra)


def _device_bytes(cache) -> int:
    return int(cache.nbytes) if isinstance(cache, PagedKVCache) else 0


class _Slot:
    """One cached conversation: its token record and the caches holding that prefix."""

    __slots__ = ("tokens", "cache", "ctx", "spilled", "sid")

    def __init__(self, tokens, cache, ctx, sid: int):
        self.tokens: list[int] = tokens
        self.cache = cache            # None while spilled
        self.ctx = ctx
        self.spilled = False
        self.sid = sid                # distinct spill file names


class PrefixCache:
    """``make_cache() -> target cache``, ``make_ctx() -> drafter context cache`` (None for
    modes without one); reuse needs at least ``min_reuse`` shared tokens; ``slots`` cached
    conversations, most recent first."""

    def __init__(self, make_cache, make_ctx=None, *, min_reuse: int = 16, l2_dir: str | None = None,
                 max_ram_bytes: int = 0, slots: int = 2):
        self.make_cache = make_cache
        self.make_ctx = make_ctx
        self.min_reuse = max(1, int(min_reuse))
        self.l2_dir = l2_dir
        self.max_ram_bytes = int(max_ram_bytes)   # device bytes of in-memory slots; 0 = never spill
        self.max_slots = max(1, int(slots))
        self.hits = 0
        self.reused_tokens = 0
        self._slots: list[_Slot] = []
        self._next_sid = 0
        if l2_dir:
            os.makedirs(l2_dir, exist_ok=True)

    # ---- public API (called under the engine's generation lock)
    def acquire(self, prompt_ids):
        """``(cache, ctx, reuse_len)``: the best slot's caches cut to the shared prefix (the
        slot is checked out until ``store``), or fresh caches and 0. At least one prompt token
        is always left to prefill, so the generation has logits to start from."""
        prompt_ids = list(prompt_ids)
        best, best_len = None, 0
        for slot in self._slots:
            reuse = max(0, min(_lcp(slot.tokens, prompt_ids), len(slot.tokens), len(prompt_ids) - 1))
            if reuse > best_len:
                best, best_len = slot, reuse
        if best is not None and best_len >= self.min_reuse:
            self._slots.remove(best)
            cache, ctx = self._materialize(best)
            if cache is not None:
                _cut(cache, best_len)
                if ctx is not None:
                    ctx.trim_to(best_len)
                self.hits += 1
                self.reused_tokens += best_len
                return cache, ctx, best_len
        return self.make_cache(), (self.make_ctx() if self.make_ctx else None), 0

    def store(self, cache, ctx, prompt_ids, token_ids) -> None:
        """Keep a finished generation's caches. They hold the prompt and every generated token
        but the last (the pending one, never fed to the target); the record claims no more
        than both caches hold, and a longer cache is cut back to the record."""
        tokens = list(prompt_ids) + list(token_ids)[:-1]
        held = _held(cache)
        if ctx is not None:
            held = min(held, int(ctx.lengths[0]))
        tokens = tokens[:held]
        _cut(cache, len(tokens))
        if ctx is not None:
            ctx.trim_to(len(tokens))
        slot = _Slot(tokens, cache, ctx, self._next_sid)
        self._next_sid += 1
        self._slots.insert(0, slot)
        while len(self._slots) > self.max_slots:
            self._evict(self._slots.pop())
        self._maybe_spill()

    def reset(self) -> None:
        self._slots = []
        self._clear_spill_files()

    def info(self) -> dict:
        newest = self._slots[0] if self._slots else None
        return {"enabled": True, "cached_tokens": len(newest.tokens) if newest else 0,
                "slots": [{"tokens": len(s.tokens), "spilled": s.spilled} for s in self._slots],
                "hits": self.hits, "reused_tokens": self.reused_tokens, "l2": bool(self.l2_dir)}

    # ---- internals
    def _materialize(self, slot: _Slot):
        if slot.cache is not None:
            return slot.cache, slot.ctx
        if slot.spilled and self.l2_dir:
            return self._load_spill(slot)
        return None, None

    def _evict(self, slot: _Slot) -> None:
        for p in self._spill_paths(slot.sid) if self.l2_dir else ():
            try:
                os.remove(p)
            except OSError:
                pass

    def _maybe_spill(self) -> None:
        if self.max_ram_bytes <= 0 or not self.l2_dir:
            return

        def total() -> int:
            return sum(_device_bytes(s.cache) + (_device_bytes(s.ctx) if s.ctx is not None else 0)
                       for s in self._slots if s.cache is not None)

        # least recent first; the newest slot spills only if it alone exceeds the budget
        for slot in reversed(self._slots):
            if total() <= self.max_ram_bytes:
                return
            if slot.cache is not None:
                self._save_spill(slot)
                slot.cache = slot.ctx = None
                slot.spilled = True

    # ---- spill files: the pages holding the first len(tokens) positions of every layer
    def _spill_paths(self, sid: int) -> tuple[str, str]:
        return (os.path.join(self.l2_dir, f"target_cache_{sid}.safetensors"),
                os.path.join(self.l2_dir, f"ctx_cache_{sid}.safetensors"))

    def _save_spill(self, slot: _Slot) -> None:
        from safetensors.torch import save_file

        tpath, cpath = self._spill_paths(slot.sid)
        meta = {"tokens": json.dumps(slot.tokens)}
        save_file(_pages_of(slot.cache, len(slot.tokens)), tpath, metadata=meta)
        if slot.ctx is not None:
            save_file(_pages_of(slot.ctx, len(slot.tokens)), cpath, metadata=meta)

    def _load_spill(self, slot: _Slot):
        from safetensors.torch import load_file

        tpath, cpath = self._spill_paths(slot.sid)
        cache = self.make_cache()
        _restore_pages(cache, load_file(tpath), len(slot.tokens))
        ctx = None
        if self.make_ctx is not None and os.path.exists(cpath):
            ctx = self.make_ctx()
            _restore_pages(ctx, load_file(cpath), len(slot.tokens))
        slot.cache, slot.ctx, slot.spilled = cache, ctx, False
        return cache, ctx

    def _clear_spill_files(self) -> None:
        if not self.l2_dir:
            return
        for p in glob.glob(os.path.join(self.l2_dir, "*_cache_*.safetensors")):
            try:
                os.remove(p)
            except OSError:
                pass


def _pools(cache: PagedKVCache) -> dict:
    out = {}
    for l in range(cache.n_layers):
        out[f"k.{l}"], out[f"v.{l}"] = cache.k[l], cache.v[l]
        if cache.k_sb[l] is not None:
            out[f"k_sb.{l}"], out[f"v_sb.{l}"] = cache.k_sb[l], cache.v_sb[l]
    return out


def _pages_of(cache: PagedKVCache, n: int) -> dict:
    """Host copies of the pages holding row 0's first n positions, per pool tensor."""
    npg = math.ceil(n / cache.page)
    idx = cache.block_table[0, :npg].to(torch.int64)
    return {k: t.index_select(0, idx).cpu().contiguous() for k, t in _pools(cache).items()}


def _restore_pages(cache: PagedKVCache, saved: dict, n: int) -> None:
    """Write spilled pages into a fresh cache's row-0 pages and set its length to n."""
    npg = math.ceil(n / cache.page)
    idx = cache.block_table[0, :npg].to(torch.int64)
    pools = _pools(cache)
    if set(saved) != set(pools):
        raise ValueError("spilled cache does not match the cache layout of make_cache()")
    for k, t in pools.items():
        src = saved[k]
        if src.shape[1:] != t.shape[1:] or src.shape[0] != npg or src.dtype != t.dtype:
            raise ValueError(f"spilled pool {k} has shape {tuple(src.shape)}, expected {npg} pages of "
                             f"{tuple(t.shape[1:])}")
        t.index_copy_(0, idx, src.to(t.device))
    cache.set_lengths([n] + [0] * (cache.B - 1))
