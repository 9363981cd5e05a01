"""Paged KV cache in HBM.

Replaces mlx_lm's KVCache / QuantizedKVCache (src/mlx_dspark/target.py:36-48 in the
reference) and the per-row BatchCache (src/mlx_dspark/batch_engine.py:61-163). One pool per
layer holds fixed pages of ``page`` tokens (layout in include/dspark_hip.h); a block table
maps each row's logical pages to physical pages, so rows can share read-only prefix pages
and roll back privately. The authoritative lengths live on the device (``seq_lens``) so a
captured HIP graph can advance and roll them back without host round trips; ``lengths``
mirrors them on the host.

The object is also a list of per-layer views with the attributes the reference's callers
read (``offset``, ``trim``, ``is_trimmable``): a decode loop that trims every layer by the
same amount (src/mlx_dspark/generate.py:928-933) trims the cache once.
"""

from __future__ import annotations

import math

import torch

from .ops import DSK_KV_BF16, DSK_KV_U8


class LayerView:
    __slots__ = ("cache", "layer")

    def __init__(self, cache: "PagedKVCache", layer: int):
        self.cache = cache
        self.layer = layer

    @property
    def offset(self) -> int:
        return self.cache.layer_offsets[self.layer]

    @offset.setter
    def offset(self, v: int) -> None:
        self.cache.layer_offsets[self.layer] = int(v)
        if self.layer == 0:
            self.cache.set_lengths([int(v)] * self.cache.B)

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(int(n), self.offset)
        self.offset = self.offset - n
        return n

    # drafter context-cache surface (src/mlx_dspark/model.py:48-80): append-only, trimmed only to
    # roll back to a shared prefix; every layer holds the same positions
    @property
    def length(self) -> int:
        return self.cache.lengths[0]

    def trim_to(self, length: int) -> None:
        if length < self.cache.lengths[0]:
            self.cache.set_lengths([int(length)] * self.cache.B)

    @property
    def keys(self):
        return self.cache.k[self.layer]

    @property
    def values(self):
        return self.cache.v[self.layer]

    @property
    def state(self):
        return self.cache.k[self.layer], self.cache.v[self.layer]


class PagedKVCache(list):
    """KV pools for ``n_layers`` layers and ``B`` rows, up to ``max_ctx`` tokens per row.
    ``spare_rows`` rows' worth of pages (and ``spare_pages`` more) sit in the pools beyond the
    rows' own pages, for block tables that point at shared or stored pages."""

    def __init__(self, n_layers: int, B: int, n_kv: int, head_dim: int, max_ctx: int, *,
                 page: int = 64, kv_bits: int | None = None, device="cuda", spare_pages: int = 0,
                 spare_rows: int = 0):
        super().__init__(LayerView(self, l) for l in range(n_layers))
        self.n_layers, self.B, self.n_kv, self.head_dim = n_layers, B, n_kv, head_dim
        self.page = page
        self.max_pages = math.ceil(max_ctx / page)
        self.max_ctx = self.max_pages * page
        self.kv_dtype = DSK_KV_U8 if kv_bits == 8 else DSK_KV_BF16
        if kv_bits not in (None, 8):
            raise ValueError(f"kv_bits={kv_bits}: only 8-bit (or None = bf16) KV is supported")
        self.n_pages = (B + spare_rows) * self.max_pages + spare_pages
        dev = torch.device(device)
        shape = (self.n_pages, n_kv, page, head_dim)
        dt = torch.uint8 if self.kv_dtype == DSK_KV_U8 else torch.bfloat16
        self.k = [torch.zeros(shape, dtype=dt, device=dev) for _ in range(n_layers)]
        self.v = [torch.zeros(shape, dtype=dt, device=dev) for _ in range(n_layers)]
        if self.kv_dtype == DSK_KV_U8:
            sbs = (self.n_pages, n_kv, page, head_dim // 64)
            self.k_sb = [torch.zeros(sbs, dtype=torch.int32, device=dev) for _ in range(n_layers)]
            self.v_sb = [torch.zeros(sbs, dtype=torch.int32, device=dev) for _ in range(n_layers)]
        else:
            self.k_sb = self.v_sb = [None] * n_layers
        self.block_table = torch.arange(B * self.max_pages, dtype=torch.int32, device=dev).view(B, self.max_pages)
        self.seq_lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.lengths = [0] * B
        self.layer_offsets = [0] * n_layers

    # ---- lengths
    def set_lengths(self, lengths) -> None:
        """Host -> device length update (eager paths; graph paths update seq_lens on device)."""
        self.lengths = [int(x) for x in lengths]
        if any(l < 0 or l > self.max_ctx for l in self.lengths):
            raise ValueError(f"cache length {self.lengths} outside [0, {self.max_ctx}]")
        self.seq_lens.copy_(torch.tensor(self.lengths, dtype=torch.int32), non_blocking=False)
        if self.B == 1:
            self.layer_offsets = [self.lengths[0]] * self.n_layers

    def note_lengths(self, lengths) -> None:
        """Record lengths the device already holds (after a device-side advance)."""
        self.lengths = [int(x) for x in lengths]
        if self.B == 1:
            self.layer_offsets = [self.lengths[0]] * self.n_layers

    @property
    def offset(self) -> int:
        return self.lengths[0]

    @property
    def length(self) -> int:
        return self.lengths[0]

    def trim_to(self, length: int) -> None:
        """Keep the first ``length`` positions of every row (K stays valid: roped at its
        absolute position)."""
        self.set_lengths([min(int(length), l) for l in self.lengths])

    def trim_rows(self, amounts) -> None:
        """Roll row b back by amounts[b] positions, clamped at zero (the batch cache's per-row
        trim, src/mlx_dspark/batch_engine.py:159-167): metadata only, so a row's next write lands
        at its new length and overwrites what was there."""
        amounts = [int(n) for n in amounts]
        if len(amounts) != self.B or min(amounts) < 0:
            raise ValueError(f"trim_rows needs {self.B} non-negative amounts, got {amounts}")
        self.set_lengths([max(0, l - n) for l, n in zip(self.lengths, amounts)])

    def check_room(self, W: int) -> None:
        if max(self.lengths) + W > self.max_ctx:
            raise ValueError(f"KV cache full: {max(self.lengths)} + {W} > {self.max_ctx} tokens")

    def layer_args(self, l: int):
        return self.k[l], self.v[l], self.k_sb[l], self.v_sb[l]

    @property
    def nbytes(self) -> int:
        t = sum(x.numel() * x.element_size() for x in self.k + self.v)
        if self.kv_dtype == DSK_KV_U8:
            t += sum(x.numel() * 4 for x in self.k_sb + self.v_sb)
        return t

    # ---- rows of a multi-row cache (continuous batching)
    def row(self, b: int) -> "RowCache":
        """A one-row cache over row b: same pools, views of row b's block table and device
        length. Every single-row op (prefill, forward, drafter ingest) runs on it unchanged."""
        return RowCache(self, b)

    def rows(self, b0: int, b1: int) -> "RowCache":
        """Rows b0 .. b1-1 seen as a B = b1 - b0 cache (a group of a batch too wide for one
        kernel pass)."""
        return RowCache(self, b0, b1)

    def row_pages(self, b: int) -> list[int]:
        return [int(x) for x in self.block_table[b].tolist()]

    def set_row_pages(self, b: int, pages: list[int]) -> None:
        """Point row b's logical pages at physical pages (shared read-only prefix pages first,
        then the row's own pages). Every entry must be a valid page of the pool."""
        if len(pages) != self.max_pages or min(pages) < 0 or max(pages) >= self.n_pages:
            raise ValueError("a block-table row needs max_pages valid page indices")
        self.block_table[b].copy_(torch.tensor(pages, dtype=torch.int32))

    def swap_rows(self, a: int, b: int) -> None:
        """Exchange two rows' block tables and lengths (slot compaction is metadata only)."""
        if a == b:
            return
        idx = torch.tensor([b, a], device=self.block_table.device)
        self.block_table[[a, b]] = self.block_table[idx]
        self.seq_lens[[a, b]] = self.seq_lens[idx]
        self.lengths[a], self.lengths[b] = self.lengths[b], self.lengths[a]

    def set_row_length(self, b: int, n: int) -> None:
        if n < 0 or n > self.max_ctx:
            raise ValueError(f"row length {n} outside [0, {self.max_ctx}]")
        self.lengths[b] = int(n)
        self.seq_lens[b].fill_(int(n))


class RowCache(PagedKVCache):
    """Rows b .. b1-1 (default: row b alone) of a PagedKVCache seen as a cache of B = b1 - b
    rows (shares the parent's pools, block-table rows and device lengths)."""

    def __init__(self, parent: PagedKVCache, b: int, b1: int | None = None):  # noqa: nothing is allocated
        list.__init__(self, (LayerView(self, l) for l in range(parent.n_layers)))
        b = int(b)
        b1 = b + 1 if b1 is None else int(b1)
        if not 0 <= b < b1 <= parent.B:
            raise ValueError(f"rows {b} .. {b1 - 1} outside the cache's {parent.B} rows")
        if isinstance(parent, RowCache):        # rows of a view: the same rows of the root cache
            b, b1, parent = parent.b + b, parent.b + b1, parent.parent
        self.parent, self.b, self.b1 = parent, b, b1
        for name in ("n_layers", "n_kv", "head_dim", "page", "max_pages", "max_ctx", "kv_dtype", "n_pages",
                     "k", "v", "k_sb", "v_sb"):
            setattr(self, name, getattr(parent, name))
        self.B = self.b1 - self.b
        self.block_table = parent.block_table[self.b:self.b1]
        self.seq_lens = parent.seq_lens[self.b:self.b1]

    @property
    def lengths(self):
        return self.parent.lengths[self.b:self.b1]

    @lengths.setter
    def lengths(self, v):
        v = [int(x) for x in v]
        if len(v) != self.B:
            raise ValueError(f"{len(v)} lengths for {self.B} rows")
        self.parent.lengths[self.b:self.b1] = v

    # row operations act on the root cache's rows (the host lengths live there)
    def swap_rows(self, a: int, b: int) -> None:
        if not (0 <= a < self.B and 0 <= b < self.B):
            raise ValueError(f"rows {a}, {b} outside the view's {self.B} rows")
        self.parent.swap_rows(self.b + a, self.b + b)

    def set_row_length(self, b: int, n: int) -> None:
        if not 0 <= b < self.B:
            raise ValueError(f"row {b} outside the view's {self.B} rows")
        self.parent.set_row_length(self.b + b, n)

    @property
    def layer_offsets(self):
        return [self.parent.lengths[self.b]] * self.n_layers

    @layer_offsets.setter
    def layer_offsets(self, v):
        pass
