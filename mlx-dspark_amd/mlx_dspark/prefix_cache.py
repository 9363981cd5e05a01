"""Prefix KV reuse across requests, on reference-counted pages of one paged arena.

Drop-in for the reference's ``PrefixCache`` surface (src/mlx_dspark/prefix_cache.py:111-175:
``acquire(prompt) -> (cache, ctx, reuse_len)``, ``store(cache, ctx, prompt, tokens)``,
``reset()``, ``info()``, the ``l2_dir`` attribute) and of ``target_cache_reusable``
(:59-76). The reference keeps a few whole per-conversation caches; this store keeps pages.

Design.
- One arena per cache kind: a B = 1 ``PagedKVCache`` whose pools hold ``1 + slots`` rows' worth
  of pages (target KV, and for DSpark the drafter's context K/V). Row 0 is the cache handed to
  the generation; every other page belongs to the store or to the free list. Page ids are per
  arena; one allocator (free stack + pin counts) runs per arena.
- The store is a tree of pages: a node is one page of one conversation, keyed by the token
  chunk it holds (``page`` tokens; a conversation's last page may hold fewer). Two
  conversations that share a prefix share the nodes, hence the physical pages, of every whole
  page of that prefix. Nothing is copied when a conversation is stored: the generation's pages
  that hold new chunks are adopted by new nodes, the rest go back to the free list.
- ``acquire`` walks the tree along the prompt. Whole matched pages are mapped read-only into
  row 0's block table and pinned (a pinned node is never evicted or spilled); the page holding
  the first position to be written, when the reuse ends inside a page, is copied into a
  private page first (copy on write: one page per layer). Row 0 gets private pages from the
  free list for everything after that.
- Eviction: ``slots`` bounds the number of stored branches (tree leaves). Past it, or when
  the free list runs short, the least recently used unpinned leaf is dropped, then its parent
  when that parent is left childless and unpinned.
- Spill (``l2_dir`` with ``max_ram_bytes`` > 0): past the byte budget of resident store pages
  the least recently used unpinned pages whose subtrees are already off the device are written
  to one safetensors file each and their pages freed; a later match reads them back into fresh
  pages before mapping them.

Positions past a row's length are never read, and every layer's K is roped at its absolute
position, so a page written by any earlier conversation is valid for every later prompt that
shares its tokens and its whole prefix.
"""

from __future__ import annotations

import glob
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


def _pool_tensors(cache: PagedKVCache) -> dict:
    """Every pool tensor of a paged cache by name; dim 0 is the physical page."""
    out = {}
    for l in range(cache.n_layers):
        out[f"k.{l}"], out[f"v.{l}"] = cache.k[l], cache.v[l]
        if cache.k_sb[l] is not None:
            out[f"ks.{l}"], out[f"vs.{l}"] = cache.k_sb[l], cache.v_sb[l]
    return out


class _Arena:
    """One paged cache plus the allocator over its physical pages."""

    def __init__(self, cache: PagedKVCache):
        if cache.B != 1:
            raise ValueError("a prefix arena is a one-row paged cache")
        self.cache = cache
        self.free = list(range(cache.n_pages - 1, -1, -1))     # stack; low page ids first
        self.pools = _pool_tensors(cache)
        self.page_bytes = sum(t[0].numel() * t.element_size() for t in self.pools.values())

    def take(self) -> int:
        return self.free.pop()

    def give(self, page: int) -> None:
        self.free.append(int(page))

    def copy_page(self, src: int, dst: int) -> None:
        for t in self.pools.values():
            t[dst].copy_(t[src])


class _Node:
    """One stored page: ``chunk`` the token ids it holds, ``pages`` its physical page in every
    arena (None while spilled), ``pins`` how many borrowed rows read it."""

    __slots__ = ("chunk", "pages", "parent", "kids", "pins", "tick", "disk", "nid")

    def __init__(self, chunk: tuple, pages, parent, nid: int):
        self.chunk = chunk
        self.pages = pages
        self.parent = parent
        self.kids: dict = {}
        self.pins = 0
        self.tick = 0
        self.disk: str | None = None
        self.nid = nid

    def depth_tokens(self) -> int:
        n, node = 0, self
        while node.parent is not None:
            n += len(node.chunk)
            node = node.parent
        return n


class PrefixCache:
    """``make_cache(spare_rows=)`` -> target paged cache, ``make_ctx(spare_rows=)`` -> drafter
    context cache (None for modes without one). Reuse needs at least ``min_reuse`` shared
    tokens; ``slots`` stored branches are kept (the arenas hold that many rows of pages)."""

    def __init__(self, make_cache, make_ctx=None, *, min_reuse: int = 16, l2_dir: str | None = None,
                 max_ram_bytes: int = 0, slots: int = 2):
        self.max_slots = max(1, int(slots))
        self.arenas = [_Arena(make_cache(spare_rows=self.max_slots))]
        if make_ctx is not None:
            self.arenas.append(_Arena(make_ctx(spare_rows=self.max_slots)))
        pages = {a.cache.page for a in self.arenas}
        if len(pages) != 1:
            raise ValueError("target and drafter-context arenas need the same page size")
        self.page = pages.pop()
        self.min_reuse = max(1, int(min_reuse))
        self.l2_dir = l2_dir
        self.max_ram_bytes = int(max_ram_bytes)
        self.hits = 0
        self.reused_tokens = 0
        self._root = _Node((), None, None, -1)
        self._clock = 0
        self._next_nid = 0
        self._out: list | None = None      # pinned nodes while row 0 is checked out
        if l2_dir:
            os.makedirs(l2_dir, exist_ok=True)

    @property
    def cache(self) -> PagedKVCache:
        return self.arenas[0].cache

    @property
    def ctx(self) -> PagedKVCache | None:
        return self.arenas[1].cache if len(self.arenas) > 1 else None

    # ------------------------------------------------------------------ public API
    def acquire(self, prompt_ids):
        """``(cache, ctx, reuse_len)``: row 0 of the arenas holding the longest stored prefix of
        the prompt (0 tokens when under ``min_reuse``). At least one prompt token is left to
        prefill, so the generation has logits to start from. The caches stay checked out
        until ``store`` (or ``reset``)."""
        if self._out is not None:
            raise RuntimeError("PrefixCache.acquire: the caches are checked out; store() or reset() first")
        ids = [int(t) for t in prompt_ids]
        path, tail, tail_len = self._match(ids)
        reuse = min(len(path) * self.page + tail_len, max(0, len(ids) - 1))
        if reuse < self.min_reuse:
            reuse, path, tail = 0, [], None
        n_shared = reuse // self.page
        cow = None
        if reuse % self.page:
            cow = path[n_shared] if n_shared < len(path) else tail
        shared = path[:n_shared]
        pinned = shared + ([cow] if cow is not None else [])
        for node in pinned:
            node.pins += 1
        taken = []                          # (arena, page): row 0's private pages so far
        try:
            for node in pinned:
                self._load(node)            # a loaded node keeps its pages: they are stored ones
            self._tick(shared[-1] if shared else None)
            if cow is not None:
                cow.tick = self._clock
            for ai, ar in enumerate(self.arenas):
                c = ar.cache
                own = self._alloc(ai, c.max_pages - n_shared)
                taken += [(ar, p) for p in own]
                if cow is not None:
                    ar.copy_page(cow.pages[ai], own[0])
                c.set_row_pages(0, [n.pages[ai] for n in shared] + own)
                c.set_lengths([reuse])
        except BaseException:
            # give back what this call took and leave row 0 empty in every arena
            for node in pinned:
                node.pins -= 1
            for ar, p in taken:
                ar.give(p)
            for ar in self.arenas:
                ar.cache.set_lengths([0])
            raise
        if cow is not None:
            cow.pins -= 1                  # its contents now live in a private page
        self._out = shared
        if reuse:
            self.hits += 1
            self.reused_tokens += reuse
        return self.cache, self.ctx, reuse

    def store(self, cache, ctx, prompt_ids, token_ids) -> None:
        """Keep a finished generation's positions. The caches hold the prompt and every
        generated token but the last (the pending one, never fed to the target); the record
        claims no more than every arena holds."""
        if self._out is None or cache is not self.cache or ctx is not self.ctx:
            raise ValueError("PrefixCache.store takes back the caches its acquire handed out")
        tokens = [int(t) for t in prompt_ids] + [int(t) for t in list(token_ids)[:-1]]
        held = min(a.cache.lengths[0] for a in self.arenas)
        tokens = tokens[:held]
        rows = [a.cache.row_pages(0) for a in self.arenas]
        for node in self._out:
            node.pins -= 1
        self._out = None
        node = self._root
        n_used = -(-len(tokens) // self.page)
        for i in range(n_used):
            chunk = tuple(tokens[i * self.page:(i + 1) * self.page])
            pages = tuple(r[i] for r in rows)
            node = self._insert(node, chunk, pages)
        for ai, ar in enumerate(self.arenas):
            for p in rows[ai][n_used:]:
                ar.give(p)
            ar.cache.set_lengths([0])
        self._tick(node if node is not self._root else None)
        self._enforce()

    def reset(self) -> None:
        """Drop every stored page and spill file, and return row 0 (checked out or not)."""
        self._root = _Node((), None, None, -1)
        self._out = None
        for ar in self.arenas:
            ar.free = list(range(ar.cache.n_pages - 1, -1, -1))
            ar.cache.set_lengths([0])
        self._clear_spill_files()

    def info(self) -> dict:
        leaves = sorted(self._leaves(), key=lambda n: -n.tick)
        nodes = list(self._nodes())
        return {"enabled": True, "cached_tokens": leaves[0].depth_tokens() if leaves else 0,
                "slots": [{"tokens": n.depth_tokens(), "spilled": self._branch_spilled(n)} for n in leaves],
                "hits": self.hits, "reused_tokens": self.reused_tokens, "l2": bool(self.l2_dir),
                "pages": {"stored": len(nodes), "resident": sum(n.pages is not None for n in nodes),
                          "shared": sum(len(n.kids) > 1 for n in nodes),
                          "free": min(len(a.free) for a in self.arenas)}}

    # ------------------------------------------------------------------ tree
    def _match(self, ids):
        """Whole-page nodes matched along ``ids``, then the best partial node below them and how
        many of its tokens match."""
        path, node, i = [], self._root, 0
        while True:
            nxt = node.kids.get(tuple(ids[i:i + self.page])) if i + self.page <= len(ids) else None
            if nxt is None or len(nxt.chunk) < self.page:
                break
            path.append(nxt)
            node, i = nxt, i + self.page
        best, best_len = None, 0
        for kid in node.kids.values():
            n = _lcp(kid.chunk, ids[i:i + self.page])
            if n > best_len:
                best, best_len = kid, n
        return path, best, best_len

    def _insert(self, node: _Node, chunk: tuple, pages: tuple) -> _Node:
        """The child of ``node`` holding ``chunk``, adopting ``pages`` when it is new (the
        caller's pages are freed when an equal or longer stored chunk already covers them)."""
        kid = node.kids.get(chunk)
        if kid is None:
            for other in node.kids.values():
                if len(other.chunk) > len(chunk) and other.chunk[:len(chunk)] == chunk:
                    kid = other            # a stored page already holds these positions
                    break
        if kid is not None:
            if kid.pages is None:          # spilled: take the resident copy instead
                self._unlink_disk(kid)
                kid.pages = pages
            elif kid.pages != pages:
                self._give(pages)
            return kid
        # shorter partial pages this chunk extends become redundant
        for key in [k for k, o in node.kids.items() if len(k) < len(chunk) and chunk[:len(k)] == k
                    and not o.kids and o.pins == 0]:
            self._drop(node.kids[key])
        kid = _Node(chunk, pages, node, self._next_nid)
        self._next_nid += 1
        node.kids[chunk] = kid
        return kid

    def _tick(self, node) -> None:
        self._clock += 1
        while node is not None and node is not self._root:
            node.tick = self._clock
            node = node.parent

    def _nodes(self):
        stack = list(self._root.kids.values())
        while stack:
            n = stack.pop()
            yield n
            stack.extend(n.kids.values())

    def _leaves(self):
        return [n for n in self._nodes() if not n.kids]

    def _branch_spilled(self, leaf: _Node) -> bool:
        node = leaf
        while node is not self._root:
            if node.pages is None:
                return True
            node = node.parent
        return False

    def _give(self, pages) -> None:
        for ai, p in enumerate(pages):
            self.arenas[ai].give(p)

    def _drop(self, node: _Node) -> None:
        """Remove an unpinned leaf and free its pages or file."""
        del node.parent.kids[node.chunk]
        if node.pages is not None:
            self._give(node.pages)
        self._unlink_disk(node)

    def _evict_one(self) -> bool:
        """Drop the least recently used unpinned leaf, then its ancestors left childless."""
        cands = [n for n in self._leaves() if n.pins == 0]
        if not cands:
            return False
        node = min(cands, key=lambda n: n.tick)
        while node is not self._root and not node.kids and node.pins == 0:
            parent = node.parent
            self._drop(node)
            node = parent
        return True

    def _alloc(self, ai: int, n: int) -> list[int]:
        ar = self.arenas[ai]
        while len(ar.free) < n:
            if not self._evict_one():
                raise RuntimeError("prefix arena has no free pages left (all stored pages are pinned)")
        return [ar.take() for _ in range(n)]

    def _enforce(self) -> None:
        while len(self._leaves()) > self.max_slots and self._evict_one():
            pass
        if self.max_ram_bytes <= 0 or not self.l2_dir:
            return
        per_page = sum(a.page_bytes for a in self.arenas)
        while True:
            resident = [n for n in self._nodes() if n.pages is not None]
            if len(resident) * per_page <= self.max_ram_bytes:
                return
            cands = [n for n in resident if n.pins == 0 and all(k.pages is None for k in n.kids.values())]
            if not cands:
                return
            self._spill(min(cands, key=lambda n: n.tick))

    # ------------------------------------------------------------------ spill files
    def _spill(self, node: _Node) -> None:
        from safetensors.torch import save_file

        path = os.path.join(self.l2_dir, f"page_{node.nid}.safetensors")
        data = {}
        for ai, ar in enumerate(self.arenas):
            for name, t in ar.pools.items():
                data[f"{ai}.{name}"] = t[node.pages[ai]].cpu().contiguous()
        save_file(data, path)
        self._give(node.pages)
        node.pages, node.disk = None, path

    def _load(self, node: _Node) -> None:
        if node.pages is not None:
            return
        from safetensors.torch import load_file

        data = load_file(node.disk)
        pages = []
        try:
            for ai, ar in enumerate(self.arenas):
                pages.append(self._alloc(ai, 1)[0])
                for name, t in ar.pools.items():
                    src = data[f"{ai}.{name}"]
                    if src.shape != t.shape[1:] or src.dtype != t.dtype:
                        raise ValueError(f"spilled page {node.disk} does not match the arena layout ({name})")
                    t[pages[-1]].copy_(src.to(t.device))
        except BaseException:
            for ai, p in enumerate(pages):      # the node stays spilled; its pages go back
                self.arenas[ai].give(p)
            raise
        node.pages = tuple(pages)
        self._unlink_disk(node)

    def _unlink_disk(self, node: _Node) -> None:
        if node.disk is not None:
            try:
                os.remove(node.disk)
            except OSError:
                pass
            node.disk = None

    def _clear_spill_files(self) -> None:
        if not self.l2_dir:
            return
        for p in glob.glob(os.path.join(self.l2_dir, "page_*.safetensors")):
            try:
                os.remove(p)
            except OSError:
                pass
