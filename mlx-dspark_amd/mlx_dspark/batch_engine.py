"""Continuous batching (drop-in for src/mlx_dspark/batch_engine.py).

Keeps the reference's surface: ``batchable``, ``batch_generate_baseline``, ``SpecSlots``
(``admit`` / ``step`` / ``has_free_slot`` / ``n_active``) and ``batch_spec_generate``
(batch_engine.py:43-55, :322-334, :431-636).

MI355X design. Every slot is one row of a paged KV cache (and of the drafter's context cache):
- per-row lengths live on the device, so rows roll back by different amounts inside the
  acceptance kernel;
- retiring a slot swaps block-table rows, so compaction copies no KV;
- a registered prompt prefix is prefilled once into spare pages, and the block tables of the
  rows that start with it point at those pages (read-only: rows only write past their prefix).

A round over the active rows is:
1. one batched drafter block forward (Markov block sampling per row);
2. one batched verify forward over [B_act, cap + 1] rows;
3. batched acceptance (greedy, or speculative sampling when temperature > 0; the reference's
   batched engine is greedy only);
4. one batched context append;
5. a single host sync.
"""

from __future__ import annotations

import time

import torch

from . import blockdraft, ops
from .generate import GenResult, _seed64
from .textstream import TextStream, eos_token_ids
from .kv import PagedKVCache

# --------------------------------------------------------------------------- capability


def batchable(target) -> bool:
    """True when the target runs the batched path: both target layouts of this engine (per-row
    lengths, block tables and sliding windows are native to its kernels; the reference falls
    back to its serial engine for gemma)."""
    if getattr(target, "is_vlm", False):
        return False
    return getattr(target, "family", "qwen3") in ("qwen3", "gemma4")


def _per_row(x, B):
    """A per-row setting given once for all rows or as one value per row."""
    return list(x) if isinstance(x, (list, tuple)) else [x] * B


class _Row:
    """The output of one batched request. It ends the way a single request ends: at an eos
    id, at ``limit`` tokens, or at a stop string (the streamer of the single-request loops).
    A round's tokens are committed whole, up to the first eos, so a row may pass its limit
    within its last round (the reference's batched rows do the same,
    src/mlx_dspark/batch_engine.py:281-291)."""

    __slots__ = ("ids", "limit", "eos", "streamer", "accepts", "done", "t0")

    def __init__(self, tokenizer, eos: set, first: int, limit: int, on_text=None, stop=None):
        self.ids = [int(first)]
        self.limit = int(limit)
        self.eos = eos
        self.streamer = TextStream(tokenizer, eos, on_text, stop)
        self.accepts: list = []
        self.t0 = time.time()
        self.done = False
        self._settle()

    def _settle(self) -> None:
        self.streamer.feed(self.ids)
        self.done = self.ids[-1] in self.eos or len(self.ids) >= self.limit or self.streamer.closed

    def extend(self, tokens, accept_len: int | None = None) -> None:
        if self.done:
            return
        if accept_len is not None:
            self.accepts.append(int(accept_len))
        for t in tokens:
            self.ids.append(int(t))
            if self.ids[-1] in self.eos:
                break
        self._settle()

    def result(self, tokenizer, seconds: float) -> GenResult:
        st = self.streamer
        st.close()
        ids = list(self.ids)
        spec = bool(self.accepts)
        rounds = list(self.accepts) if spec else [1] * len(ids)
        reason = st.finish_reason(ids, self.limit, ids[-1])
        return GenResult(text=st.result_text(ids), token_ids=ids, num_tokens=len(ids),
                         num_rounds=len(rounds), accept_lengths=rounds,
                         target_forwards=len(rounds) + 1 if spec else len(ids), seconds=seconds,
                         finish_reason=reason)


# --------------------------------------------------------------------------- baseline


def batch_generate_baseline(target, tokenizer, prompts_ids, *, max_new_tokens=128, temperature: float = 0.0,
                            top_p: float = 1.0, top_k: int = 0, on_texts=None, stops=None, seed=None,
                            max_ctx: int | None = None) -> list:
    """Static batched plain decode of B prompts (batch_engine.py:322-370): every row advances
    one token per step through one shared forward; finished rows keep stepping (output
    ignored) until all finish. Returns one GenResult per row."""
    B = len(prompts_ids)
    if B == 0:
        return []
    model = target.model
    dev = model.device
    mnt = _per_row(max_new_tokens, B)
    need = max(len(p) for p in prompts_ids) + max(mnt) + 8
    cache = target.make_cache(B=B, max_ctx=max(max_ctx or 0, need))
    s64 = _seed64(seed)
    t0 = time.time()
    last = torch.empty((B, model.args.vocab_size), dtype=torch.float32, device=dev)
    for b, ids in enumerate(prompts_ids):
        lg, _ = model.prefill(list(ids), cache.row(b))
        last[b].copy_(lg[0, -1])
    tok, _ = ops.sample_rows(last, temperature, top_p, top_k, seed=s64, offset=0)
    eos = eos_token_ids(tokenizer)
    ot, sp = _per_row(on_texts, B), _per_row(stops, B)
    rows = [_Row(tokenizer, eos, t, mnt[b], ot[b], sp[b]) for b, t in enumerate(tok.tolist())]
    cur = tok.view(B, 1).to(torch.int32)
    step = 1
    while not all(r.done for r in rows):
        lg, _ = model.forward(cur, cache, None)
        tok, _ = ops.sample_rows(lg[:, -1].contiguous(), temperature, top_p, top_k, seed=s64, offset=step)
        step += 1
        for r, t in zip(rows, tok.tolist()):
            r.extend([t])
        cur = tok.view(B, 1).to(torch.int32)
    secs = time.time() - t0
    return [r.result(tokenizer, secs) for r in rows]


# --------------------------------------------------------------------------- spec slots


class SpecSlots:
    """Fixed-capacity continuous batched DSpark speculative decoding (batch_engine.py:431-598).

    ``capacity`` slots share one paged target cache and one paged drafter-context cache; a
    request is :meth:`admit`-ted into the next free slot (single-row prefill into that row),
    :meth:`step` runs one speculative round over every active row, and a finished row is
    retired at once: its result is returned and the last active row's block-table row moves
    into its place, so the active rows stay a prefix 0 .. n_active-1 and every forward runs at
    the active width.

    Greedy (temperature 0) output per row is the target's greedy decoding. With temperature
    > 0, rows use speculative sampling (min(1, p/q) acceptance, residual resample), with
    Philox streams keyed by (seed, round). ``register_prefix`` prefills a shared prompt
    prefix once; admitted prompts that start with it reuse its KV pages."""

    def __init__(self, target, tokenizer, drafter, *, capacity: int, max_draft_tokens: int = 2,
                 batched_drafter: bool = True, cap_controller=None, temperature: float = 0.0, top_p: float = 1.0,
                 top_k: int = 0, seed=None, max_ctx: int = 16384, prefix_pages: int = 0):
        cfg = drafter.config
        self.target, self.tokenizer, self.drafter = target, tokenizer, drafter
        self.model = target.model
        self.dev = self.model.device
        self.tap = list(cfg.target_layer_ids)
        self.k = int(cfg.block_size)
        self.mask_id = int(cfg.mask_token_id)
        self.cap = max(1, min(int(max_draft_tokens), self.k))
        self.ctrl = cap_controller
        self.batched_drafter = batched_drafter
        self.capacity = int(capacity)
        # any capacity: batches of more than 64 rows run as groups of whole rows per kernel pass
        if self.capacity < 1 or max(self.k, self.cap + 1) > 64:
            raise ValueError(f"capacity {capacity} / block {max(self.k, self.cap + 1)}: a block is at most 64 rows")
        self.temperature, self.top_p, self.top_k = float(temperature), float(top_p), int(top_k)
        self.s64 = _seed64(seed)
        self.round = 0
        # one row per slot, plus spare pages for registered prefixes
        a, c = self.model.args, drafter.config
        self.cache = PagedKVCache(a.num_hidden_layers, self.capacity, a.num_key_value_heads, a.head_dim, max_ctx,
                                  kv_bits=target.kv_bits, device=self.dev, spare_pages=prefix_pages)
        da = drafter.args    # the drafter's own attention shape (gemma4: the global kv heads)
        self.ctx = PagedKVCache(c.num_hidden_layers, self.capacity, da.num_key_value_heads, da.head_dim,
                                max_ctx + c.block_size, device=self.dev, spare_pages=prefix_pages)
        self._spare_next = 0
        self.prefixes: list = []          # (token tuple, target pages, drafter pages)
        self.n_active = 0
        C = self.capacity
        self.pending = [0] * C
        self.rows: list = [None] * C
        self.meta = [None] * C
        self.eos = eos_token_ids(tokenizer)
        # own page range of each slot (moves with the slot's block-table row on compaction)
        self.range_t = [self.cache.row_pages(b) for b in range(C)]
        self.range_d = [self.ctx.row_pages(b) for b in range(C)]

    @property
    def has_free_slot(self) -> bool:
        return self.n_active < self.capacity

    # ---------------------------------------------------------------- prefixes
    def register_prefix(self, prefix_ids) -> int:
        """Prefill a shared prefix once into spare pages (target KV and drafter context). Only
        whole pages are shared; returns the shared length in tokens."""
        page = self.cache.page
        n = (len(prefix_ids) // page) * page
        npg = n // page
        if n == 0:
            return 0
        spare0 = self.capacity * self.cache.max_pages
        if self._spare_next + npg > self.cache.n_pages - spare0 or \
                self._spare_next + npg > self.ctx.n_pages - self.capacity * self.ctx.max_pages:
            raise ValueError("not enough spare pages for this prefix (raise prefix_pages)")
        tp = [spare0 + self._spare_next + i for i in range(npg)]
        dp = [self.capacity * self.ctx.max_pages + self._spare_next + i for i in range(npg)]
        self._spare_next += npg
        # prefill through slot 0's row with its table pointing at the spare pages
        b = 0
        saved_t, saved_d = self.cache.row_pages(b), self.ctx.row_pages(b)
        lt, ld = self.cache.lengths[b], self.ctx.lengths[b]
        self.cache.set_row_pages(b, tp + saved_t[npg:])
        self.ctx.set_row_pages(b, dp + saved_d[npg:])
        self.cache.set_row_length(b, 0)
        self.ctx.set_row_length(b, 0)
        rc, rd = self.cache.row(b), self.ctx.row(b)
        self.model.prefill(list(prefix_ids[:n]), rc, self.tap,
                           on_chunk=lambda fused, pos: self.drafter.update_context(fused, pos, rd))
        self.cache.set_row_pages(b, saved_t)
        self.ctx.set_row_pages(b, saved_d)
        self.cache.set_row_length(b, lt)
        self.ctx.set_row_length(b, ld)
        self.prefixes.append((tuple(int(t) for t in prefix_ids[:n]), tp, dp))
        return n

    def _match_prefix(self, ids):
        best = None
        for toks, tp, dp in self.prefixes:
            n = len(toks)
            if n < len(ids) and tuple(ids[:n]) == toks and (best is None or n > len(best[0])):
                best = (toks, tp, dp)
        return best

    # ---------------------------------------------------------------- admission
    def admit(self, prompt_ids, *, max_new_tokens: int, on_text=None, stop=None, meta=None) -> None:
        """Prefill one request into the next free slot (batch_engine.py:472-500)."""
        if not self.has_free_slot:
            raise RuntimeError("SpecSlots.admit: no free slot")
        ids = [int(t) for t in prompt_ids]
        b = self.n_active
        own_t, own_d = self.range_t[b], self.range_d[b]
        hit = self._match_prefix(ids)
        n0 = 0
        if hit is not None:
            toks, tp, dp = hit
            n0 = len(toks)
            self.cache.set_row_pages(b, tp + own_t[len(tp):])
            self.ctx.set_row_pages(b, dp + own_d[len(dp):])
        else:
            self.cache.set_row_pages(b, own_t)
            self.ctx.set_row_pages(b, own_d)
        self.cache.set_row_length(b, n0)
        self.ctx.set_row_length(b, n0)
        rc, rd = self.cache.row(b), self.ctx.row(b)
        rc.check_room(len(ids) - n0 + self.k + 1)
        logits, _ = self.model.prefill(ids[n0:], rc, self.tap,
                                       on_chunk=lambda fused, pos: self.drafter.update_context(fused, pos, rd))
        tok, _ = ops.sample_rows(logits[0, -1:].contiguous(), self.temperature, self.top_p, self.top_k,
                                 seed=self.s64, offset=0xFFFFFFFF)
        first = int(tok.item())
        self.pending[b] = first
        self.rows[b] = _Row(self.tokenizer, self.eos, first, max_new_tokens, on_text, stop)
        self.meta[b] = meta
        self.n_active += 1

    def _retire(self, b: int):
        meta, res = self.meta[b], self.rows[b].result(self.tokenizer, time.time() - self.rows[b].t0)
        last = self.n_active - 1
        if b != last:
            self.cache.swap_rows(b, last)
            self.ctx.swap_rows(b, last)
            for st in (self.pending, self.rows, self.meta, self.range_t, self.range_d):
                st[b], st[last] = st[last], st[b]
        self.cache.set_row_length(last, 0)
        self.ctx.set_row_length(last, 0)
        self.rows[last], self.meta[last], self.pending[last] = None, None, 0
        self.n_active = last
        return meta, res

    def _sweep_finished(self) -> list:
        out = []
        b = 0
        while b < self.n_active:
            if self.rows[b].done:
                out.append(self._retire(b))
            else:
                b += 1
        return out

    # ---------------------------------------------------------------- one round
    def step(self) -> list:
        """One speculative round over the active rows; returns [(meta, GenResult), ...] for the
        requests that finished (already retired)."""
        finished = self._sweep_finished()
        B = self.n_active
        if B == 0:
            return finished
        cap = self.cap if self.ctrl is None else max(
            1, min(self.ctrl.cap_for(B) if (B > 1 and hasattr(self.ctrl, "cap_for")) else self.ctrl.cap, self.k))
        W = cap + 1
        for b in range(B):
            self.cache.row(b).check_room(W)
            self.ctx.row(b).check_room(W + self.k)
        d, dev = self.drafter, self.dev
        sampled = self.temperature > 0.0
        pend = torch.tensor(self.pending[:B], dtype=torch.int32, device=dev)
        block = torch.full((B, self.k), self.mask_id, dtype=torch.int32, device=dev)
        block[:, 0] = pend
        # ---- 1. draft
        if self.batched_drafter:
            base = d.block_logits(block, self.ctx, cap)                                  # [B, cap, V]
        else:
            base = torch.cat([d.block_logits(block[b:b + 1], self.ctx.row(b), cap) for b in range(B)])
        q_logits = None
        if sampled:
            drafts, q_logits = d.sample_block_probs(base, pend, self.temperature, self.top_p, self.top_k,
                                                    seed=self.s64, offset=self.round)
        else:
            drafts = d.sample_block(base, pend)                                          # [B, cap]
        # ---- 2. batched verify at the active width
        vids = torch.cat([pend.view(B, 1), drafts.view(B, cap)], dim=1).contiguous()
        v_logits, v_fused = self.model.forward(vids, self.cache, self.tap, advance=False)
        # ---- 3. acceptance (advances each row's length by n + 1)
        n_t = torch.empty(B, dtype=torch.int32, device=dev)
        tok_t = torch.empty(B, dtype=torch.int32, device=dev)
        seq = self.cache.seq_lens[:B]
        if sampled:
            ops.accept_sample(v_logits, q_logits, drafts.view(B, cap).contiguous(), self.temperature, self.top_p,
                              self.top_k, q_mul_inv_t=True, seed=self.s64, offset=self.round, seq_lens=seq,
                              n_out=n_t, token_out=tok_t)
        else:
            ops.accept_greedy(v_logits, drafts.view(B, cap).contiguous(), seq_lens=seq, n_out=n_t, token_out=tok_t)
        # ---- 4. drafter context: each row keeps its n + 1 committed positions
        blockdraft.ingest_rows(d, v_fused, self.ctx, n_t)
        self.round += 1
        n_list, tok_list, dr = n_t.tolist(), tok_t.tolist(), drafts.view(B, cap).tolist()
        for b in range(B):
            n = int(n_list[b])
            committed = [int(x) for x in dr[b][:n]] + [int(tok_list[b])]
            self.cache.lengths[b] += n + 1
            self.ctx.lengths[b] += n + 1
            self.rows[b].extend(committed, accept_len=len(committed))
            self.pending[b] = self.rows[b].ids[-1]
            if self.ctrl is not None:
                self.ctrl.update(n, cap)
        return finished + self._sweep_finished()


def batch_spec_generate(target, tokenizer, drafter, prompts_ids, *, max_new_tokens=128, max_draft_tokens: int = 2,
                        batched_drafter: bool = True, on_texts=None, stops=None, seed=None, temperature: float = 0.0,
                        top_p: float = 1.0, top_k: int = 0, max_ctx: int | None = None) -> list:
    """Static batched DSpark speculative decoding (batch_engine.py:601-636): admit all B
    prompts into a SpecSlots of capacity B and step until done; results in prompt order."""
    B = len(prompts_ids)
    if B == 0:
        return []
    mnt = _per_row(max_new_tokens, B)
    ot, sp = _per_row(on_texts, B), _per_row(stops, B)
    k = int(drafter.config.block_size)
    need = max(len(p) for p in prompts_ids) + max(mnt) + 2 * k + 8
    slots = SpecSlots(target, tokenizer, drafter, capacity=B, max_draft_tokens=max_draft_tokens,
                      batched_drafter=batched_drafter, temperature=temperature, top_p=top_p, top_k=top_k, seed=seed,
                      max_ctx=max(max_ctx or 0, need))
    for i, ids in enumerate(prompts_ids):
        slots.admit(ids, max_new_tokens=mnt[i], on_text=ot[i], stop=sp[i], meta=i)
    results: list = [None] * B
    while slots.n_active:
        for meta, res in slots.step():
            results[meta] = res
    return results
