"""Speculative decoding loops (drop-in for the reference's generate.py API).

``speculative_generate`` (DSpark drafter), ``dflash_generate`` (DFlash drafter) and
``greedy_generate`` keep the reference's signatures and ``GenResult`` (src/mlx_dspark/
generate.py:27-46, :373-392, :468-485, :691-718). A round is: draft a block, verify it in one
target forward, accept the matching prefix plus one token, roll the KV back to the accepted
length and grow the drafter context.

On this engine the whole greedy round runs on the device with static buffers: the draft
never visits the host before verify, acceptance and rollback update device-side lengths,
and from the second round on the round is one replay of a captured HIP graph followed by a
single host sync that reads (n, token, draft). Sampled rounds (temperature > 0) run the same
kernels eagerly, with Philox uniforms keyed by ``seed`` and the round number.
"""

from __future__ import annotations

import collections
import time
from dataclasses import dataclass

import torch

from . import blockdraft, ops
from .textstream import StopStreaming, TextStream, encode_messages, encode_prompt, eos_token_ids  # noqa: F401

# ============================================================================ results
@dataclass
class GenResult:
    text: str
    token_ids: list
    num_tokens: int
    num_rounds: int
    accept_lengths: list
    target_forwards: int
    seconds: float
    finish_reason: str = "stop"
    lookup_rounds: int = 0
    logprobs: list | None = None

    @property
    def mean_accept_len(self) -> float:
        return self.num_tokens / max(self.num_rounds, 1)

    @property
    def tokens_per_sec(self) -> float:
        return self.num_tokens / max(self.seconds, 1e-9)


# ============================================================================ sampling helpers
def _pick(logits_row: torch.Tensor, temperature: float, top_p=1.0, top_k=0, seed=0, offset=0xFFFFFFFF) -> int:
    """argmax (T == 0) or a truncated sample of one logits row (one host sync)."""
    tok, _ = ops.sample_rows(logits_row.reshape(1, -1).float(), temperature, top_p, top_k, seed=seed, offset=offset)
    return int(tok.item())


def _seed64(seed) -> int:
    return 0x5EED if seed is None else int(seed) & ((1 << 64) - 1)


def _logprobs_for_block(logits_rows: torch.Tensor, token_ids, top_k: int) -> list:
    """Per-token logprobs of the committed tokens from the raw target logits rows [P, V] at
    their positions: [{token_id, logprob, top: [(id, logprob), ...]}] of log_softmax (the
    target's own distribution, independent of temperature and penalties; top_k 0 = chosen
    token only; ties ordered by token id). One device kernel, one host sync
    (src/mlx_dspark/generate.py:149-176)."""
    P = len(token_ids)
    if P == 0:
        return []
    top_k = max(0, min(int(top_k or 0), logits_rows.shape[-1]))
    if top_k > 64:
        raise ValueError(f"logprobs={top_k}: at most 64 alternatives per token")
    toks = torch.tensor([int(t) for t in token_ids], dtype=torch.int32, device=logits_rows.device)
    chosen, ids, vals = ops.row_logprobs(logits_rows[:P], toks, top_k)
    ch = chosen.tolist()
    if top_k:
        ids, vals = ids.tolist(), vals.tolist()
    out = []
    for i in range(P):
        e = {"token_id": int(token_ids[i]), "logprob": float(ch[i])}
        if top_k:
            e["top"] = [(int(t), float(v)) for t, v in zip(ids[i], vals[i])]
        out.append(e)
    return out


# ============================================================================ greedy baseline
def greedy_generate(target_model, tokenizer, prompt: str = "", *, prompt_ids=None, cache=None, reuse_len: int = 0,
                    max_new_tokens: int = 128, temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0,
                    presence_penalty: float = 0.0, frequency_penalty: float = 0.0, logprobs=None, seed=None,
                    apply_chat_template: bool = True, stop=None, on_text=None) -> GenResult:
    """Plain one-token-per-forward decoding of the target (src/mlx_dspark/generate.py:373-465)."""
    eos_ids = eos_token_ids(tokenizer)
    ids = prompt_ids if prompt_ids is not None else encode_prompt(tokenizer, prompt, apply_chat_template)
    if cache is None:
        cache = target_model.make_cache()
        reuse_len = 0
    st = TextStream(tokenizer, eos_ids, on_text, stop)
    s64 = _seed64(seed)
    pen = _Penalizer(presence_penalty, frequency_penalty)
    lp_list: list | None = [] if logprobs is not None else None
    t0 = time.time()
    model = target_model.model
    logits, _ = model.prefill(ids[reuse_len:] if reuse_len else ids, cache)
    row = logits[0, -1:]
    out_ids: list = []
    cur = torch.empty((1, 1), dtype=torch.int32, device=model.device)
    step = 0
    while True:
        # penalties see every token emitted so far; logprobs read the raw row
        picked = pen.apply(row.clone(), []) if pen.active else row
        nxt = _pick(picked[0], temperature, top_p, top_k, s64, step)
        step += 1
        out_ids.append(nxt)
        pen.add([nxt])
        if lp_list is not None:
            lp_list.extend(_logprobs_for_block(row, [nxt], logprobs))
        st.feed(out_ids)
        if len(out_ids) >= max_new_tokens or nxt in eos_ids or st.closed:
            break
        cur.fill_(nxt)
        lg, _ = model.forward(cur, cache, None)
        row = lg[0, -1:]
    st.close()
    secs = time.time() - t0
    return GenResult(text=st.result_text(out_ids), token_ids=out_ids, num_tokens=len(out_ids),
                     num_rounds=len(out_ids), accept_lengths=[1] * len(out_ids), target_forwards=len(out_ids),
                     seconds=secs, finish_reason=st.finish_reason(out_ids, max_new_tokens, nxt),
                     logprobs=lp_list)


# ============================================================================ DFlash
class _DFlashRound:
    """Static buffers and the device-side body of one DFlash round (greedy or sampled)."""

    def __init__(self, target, drafter, cache, dcache, cap: int, temperature: float, top_p: float, top_k: int,
                 seed: int):
        self.target, self.drafter, self.cache, self.dcache = target, drafter, cache, dcache
        self.model = target.model
        cfg = drafter.config
        self.tap = list(cfg.target_layer_ids)
        self.bs = int(cfg.block_size)
        self.cap = cap
        self.T, self.top_p, self.top_k, self.seed = temperature, top_p, top_k, seed
        dev = self.model.device
        V = self.model.args.vocab_size
        H = self.model.args.hidden_size
        self.block = torch.full((1, self.bs), int(cfg.mask_token_id), dtype=torch.int32, device=dev)
        # one id buffer [n, token, draft...]: the verify ids [pending] + draft are its tail, and
        # acceptance writes the next round's pending over this round's: no copies between steps
        self.out = torch.zeros(2 + cap, dtype=torch.int32, device=dev)
        self.n, self.pending, self.draft = self.out[0:1], self.out[1:2], self.out[2:]
        self.token = self.pending
        self.verify = self.out[1:].view(1, cap + 1)
        self.head = torch.empty((cap, V), dtype=torch.float32, device=dev)
        self.v_logits = torch.empty((cap + 1, V), dtype=torch.float32, device=dev)
        self.v_fused = torch.empty((cap + 1, len(self.tap) * H), dtype=torch.bfloat16, device=dev)
        self.tt = torch.zeros((1, cap + 1), dtype=torch.int32, device=dev)
        # sampled rounds: the draft distribution, and the round's Philox offset as a device
        # word (written before each call, so one captured graph serves every round)
        self.q_probs = torch.empty((cap, V), dtype=torch.float32, device=dev) if temperature > 0 else None
        self.rng_off = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graph = None
        self.calls = 0
        # src: a partner round's pending slot this round copies its own from on the device
        # (_DFlashPipe); the round's ids land in pinned host memory, ready at `ready`
        self.src = None
        self.host_out = torch.zeros(2 + cap, dtype=torch.int32, pin_memory=True)
        self.ready = torch.cuda.Event()

    def body(self) -> None:
        if self.src is not None:
            self.pending.copy_(self.src)
        self.block[0, 0:1].copy_(self.pending)
        self.drafter.block_logits(self.block, self.dcache, 1, self.cap, out=self.head)
        if self.T > 0:
            ops.sample_rows(self.head, self.T, self.top_p, self.top_k, seed=self.seed, token_out=self.draft,
                            probs_out=self.q_probs, offset_dev=self.rng_off)
        else:
            ops.sample_rows(self.head, 0.0, token_out=self.draft)
        self.model.forward(self.verify, self.cache, self.tap, advance=False, logits_out=self.v_logits,
                           fused_out=self.v_fused)
        if self.T > 0:
            ops.accept_sample(self.v_logits.view(1, self.cap + 1, -1), self.head.view(1, self.cap, -1),
                              self.draft.view(1, -1), self.T, self.top_p, self.top_k, seed=self.seed,
                              seq_lens=self.cache.seq_lens, n_out=self.n, token_out=self.token,
                              offset_dev=self.rng_off)
        else:
            ops.accept_greedy(self.v_logits.view(1, self.cap + 1, -1), self.draft.view(1, -1),
                              seq_lens=self.cache.seq_lens, tt=self.tt, n_out=self.n, token_out=self.token)
        self.drafter.ingest(self.v_fused, self.dcache, n_valid=self.n)     # commit [anchor, accepted]

    def launch(self, round_idx: int, use_graph: bool) -> None:
        """Enqueue the round: the first of this width runs eagerly (it sizes the workspaces),
        later ones replay one captured graph; then the ids' copy to host memory."""
        if self.T > 0:                                               # greedy rounds draw nothing
            self.rng_off.fill_(round_idx & 0x7FFFFFFF)
        if use_graph:
            if self.graph is None and self.calls >= 1:
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph):
                    self.body()
            if self.graph is not None:
                self.graph.replay()
            else:
                self.body()
        else:
            self.body()
        self.calls += 1
        self.host_out.copy_(self.out, non_blocking=True)
        self.ready.record()

    def result(self):
        """(n, token, draft) of the last launch: waits for it alone, then records the lengths
        the device already advanced."""
        self.ready.synchronize()
        o = self.host_out.tolist()
        n, token, draft = o[0], o[1], o[2:]
        self.cache.note_lengths([self.cache.lengths[0] + n + 1])
        self.dcache.note_lengths([self.dcache.lengths[0] + n + 1])
        return n, token, draft

    def run(self, round_idx: int, use_graph: bool):
        self.launch(round_idx, use_graph)
        return self.result()                                          # the round's one host sync


class _DFlashPipe:
    """Rounds of one width enqueued one ahead of the host: two _DFlashRound objects alternate,
    each reading its pending token from the other's output on the device, so the next round is
    on the GPU while the host reads this one's ids, checks the stop conditions and streams text
    (one round at a time, the GPU sat idle meanwhile). The rounds and their inputs are the
    sequential loop's; a round enqueued past the end of a generation is undone by restoring the
    caches' lengths (its KV writes lie past them)."""

    def __init__(self, target, drafter, cache, dcache, cap: int, temperature: float, top_p: float, top_k: int,
                 seed: int, use_graph: bool = True):
        self.rounds = [_DFlashRound(target, drafter, cache, dcache, cap, temperature, top_p, top_k, seed)
                       for _ in range(2)]
        self.rounds[0].src = self.rounds[1].pending
        self.rounds[1].src = self.rounds[0].pending
        self.cache, self.dcache, self.W = cache, dcache, cap + 1
        self.use_graph = use_graph
        self.queue: collections.deque = collections.deque()
        self.turn = 0
        self.next_idx = 0

    def start(self, pending: int, round_idx: int = 0) -> None:
        """The first round's pending token (its source slot) and Philox round index."""
        self.rounds[1 - self.turn].pending.fill_(pending)
        self.next_idx = round_idx

    def room(self, rounds: int) -> bool:
        """Whether `rounds` more rounds fit both caches (host lengths: rounds collected so far)."""
        return (self.cache.lengths[0] + rounds * self.W <= self.cache.max_ctx
                and self.dcache.lengths[0] + rounds * self.W <= self.dcache.max_ctx)

    def enqueue(self) -> None:
        rnd = self.rounds[self.turn]
        self.turn ^= 1
        rnd.launch(self.next_idx, self.use_graph)
        self.next_idx += 1
        self.queue.append(rnd)

    def collect(self):
        """(n, token, draft) of the oldest enqueued round."""
        return self.queue.popleft().result()

    def cancel(self) -> None:
        """Undo the rounds still enqueued: the caches go back to the collected lengths."""
        if self.queue:
            self.queue.clear()
            self.cache.set_lengths(self.cache.lengths)
            self.dcache.set_lengths(self.dcache.lengths)


def dflash_generate(target_model, tokenizer, drafter, prompt: str = "", *, prompt_ids=None, max_new_tokens: int = 128,
                    max_draft_tokens=None, cap_controller=None, temperature: float = 0.0, top_p: float = 1.0,
                    top_k: int = 0, apply_chat_template: bool = True, seed=None, stop=None, on_text=None,
                    use_graph: bool = True, max_ctx: int | None = None) -> GenResult:
    """Speculative decoding with a DFlash block-diffusion drafter (src/mlx_dspark/generate.py:468-601)."""
    if getattr(drafter, "embed_tokens", None) is None:
        drafter.bind(target_model.model)
    cfg = drafter.config
    tap = list(cfg.target_layer_ids)
    kdraft = int(cfg.block_size) - 1
    cap = kdraft if max_draft_tokens is None else max(1, min(int(max_draft_tokens), kdraft))
    eos_ids = eos_token_ids(tokenizer)
    ids = prompt_ids if prompt_ids is not None else encode_prompt(tokenizer, prompt, apply_chat_template)
    need = len(ids) + max_new_tokens + 2 * (cap + 1) + 8
    max_ctx = max(max_ctx or 0, need)
    cache = target_model.make_cache(max_ctx=max_ctx)
    dcache = drafter.make_cache(max_ctx=max_ctx)
    st = TextStream(tokenizer, eos_ids, on_text, stop)
    s64 = _seed64(seed)
    t0 = time.time()

    logits, fused = target_model.model.prefill(ids, cache, tap)
    drafter.ingest(fused, dcache)                                     # whole prompt -> draft context
    pending = _pick(logits[0, -1], temperature, top_p, top_k, s64, 0xFFFFFFFF)
    out_ids = [pending]
    accept_lengths: list = []
    target_forwards = 1
    # one round object (static buffers, captured graph) per verify width: a cap controller may
    # pick a different cap every round (generate.py:537-538)
    rounds: dict = {}
    st.feed(out_ids)
    r = 0
    if use_graph and cap_controller is None:
        # a fixed width: each round enqueued before the host reads the previous one
        pipe = _DFlashPipe(target_model, drafter, cache, dcache, cap, temperature, top_p, top_k, s64)
        pipe.start(pending)
        going = len(out_ids) < max_new_tokens and pending not in eos_ids and not st.closed
        if going and pipe.room(1):
            pipe.enqueue()
        while pipe.queue:
            if len(pipe.queue) == 1 and pipe.room(2):
                pipe.enqueue()
            n, token, draft = pipe.collect()
            committed = draft[:n] + [token]
            target_forwards += 1
            accept_lengths.append(len(committed))
            for tok in committed:
                out_ids.append(tok)
                if tok in eos_ids:
                    break
            pending = out_ids[-1]
            st.feed(out_ids)
            if not (len(out_ids) < max_new_tokens and pending not in eos_ids and not st.closed):
                pipe.cancel()
                break
            if not pipe.queue and pipe.room(1):
                pipe.enqueue()
    while (not use_graph or cap_controller is not None) and len(out_ids) < max_new_tokens \
            and pending not in eos_ids and not st.closed:
        c = cap if cap_controller is None else max(1, min(int(cap_controller.cap), cap))
        if cache.lengths[0] + c + 1 > cache.max_ctx:
            break
        rnd = rounds.get(c)
        if rnd is None:
            rnd = rounds[c] = _DFlashRound(target_model, drafter, cache, dcache, c, temperature, top_p, top_k, s64)
        rnd.pending.fill_(pending)
        n, token, draft = rnd.run(r, use_graph)
        r += 1
        if cap_controller is not None:
            cap_controller.update(n, len(draft))
        committed = draft[:n] + [token]
        target_forwards += 1
        accept_lengths.append(len(committed))
        for tok in committed:
            out_ids.append(tok)
            if tok in eos_ids:
                break
        pending = out_ids[-1]
        st.feed(out_ids)
    st.close()
    secs = time.time() - t0
    return GenResult(text=st.result_text(out_ids), token_ids=out_ids, num_tokens=len(out_ids),
                     num_rounds=len(accept_lengths), accept_lengths=accept_lengths, target_forwards=target_forwards,
                     seconds=secs, finish_reason=st.finish_reason(out_ids, max_new_tokens, pending))


# ============================================================================ penalties
class _Penalizer:
    """OpenAI presence / frequency penalties on the target's verify logits (the behaviour of
    the reference's _Penalizer, src/mlx_dspark/generate.py:179-228): row i of a verify block
    subtracts presence * (count > 0) + frequency * count over the completion tokens so far
    plus the block's own draft prefix draft[:i]. Inactive (both 0) it is a no-op."""

    def __init__(self, presence: float = 0.0, frequency: float = 0.0):
        self.presence = float(presence or 0.0)
        self.frequency = float(frequency or 0.0)
        self.active = bool(self.presence or self.frequency)
        self.counts: dict = {}

    def add(self, tokens) -> None:
        if self.active:
            for t in tokens:
                self.counts[int(t)] = self.counts.get(int(t), 0) + 1

    def block_rows(self, draft_prefix) -> list:
        """[{token: penalty}] for the len(draft_prefix) + 1 rows of a verify block."""
        base = {t: self.presence + self.frequency * c for t, c in self.counts.items()}
        rows = [base]
        seen = dict(self.counts)
        for d in draft_prefix:
            d = int(d)
            nxt = dict(rows[-1])
            nxt[d] = nxt.get(d, 0.0) + self.frequency + (self.presence if seen.get(d, 0) == 0 else 0.0)
            seen[d] = seen.get(d, 0) + 1
            rows.append(nxt)
        return rows

    def apply(self, v_logits: torch.Tensor, draft_prefix) -> torch.Tensor:
        """Penalise v_logits [len(draft)+1, V] (f32, device) in place; identity when inactive."""
        if not self.active:
            return v_logits
        rows = self.block_rows(draft_prefix)
        ptr, ids, vals = [0], [], []
        for r in rows:
            for t, v in r.items():
                if v:
                    ids.append(t)
                    vals.append(v)
            ptr.append(len(ids))
        if not ids:
            return v_logits
        dev = v_logits.device
        ops.logits_penalize(v_logits, torch.tensor(ptr, dtype=torch.int32, device=dev),
                            torch.tensor(ids, dtype=torch.int32, device=dev),
                            torch.tensor(vals, dtype=torch.float32, device=dev))
        return v_logits


# ============================================================================ DSpark
class _DSparkRound:
    """Static buffers and the device-side body of a greedy DSpark round at a fixed cap: draft
    the block, Markov-sample cap tokens, verify [pending] + draft, accept, roll back, grow the
    drafter context. Replayed as one HIP graph from its second use on."""

    def __init__(self, target, drafter, cache, dcache, cap: int):
        self.target, self.drafter, self.cache, self.dcache = target, drafter, cache, dcache
        self.model = target.model
        cfg = drafter.config
        self.tap = list(cfg.target_layer_ids)
        self.k = int(cfg.block_size)
        self.cap = cap
        dev = self.model.device
        V, H = self.model.args.vocab_size, self.model.args.hidden_size
        self.block = torch.full((1, self.k), int(cfg.mask_token_id), dtype=torch.int32, device=dev)
        # one id buffer [n, token, draft...] (as in _DFlashRound): verify ids = its tail
        self.out = torch.zeros(2 + cap, dtype=torch.int32, device=dev)
        self.n, self.pending = self.out[0:1], self.out[1:2]
        self.draft = self.out[2:].view(1, cap)
        self.token = self.pending
        self.verify = self.out[1:].view(1, cap + 1)
        self.head = torch.empty((cap, drafter.lm_head.N), dtype=torch.float32, device=dev)
        self.v_logits = torch.empty((cap + 1, V), dtype=torch.float32, device=dev)
        self.v_fused = torch.empty((cap + 1, len(self.tap) * H), dtype=torch.bfloat16, device=dev)
        self.tt = torch.zeros((1, cap + 1), dtype=torch.int32, device=dev)
        self.graph = None
        self.calls = 0
        self.uses = 0

    def body(self) -> None:
        self.block[0, 0:1].copy_(self.pending)
        self.drafter.block_logits(self.block, self.dcache, self.cap, out=self.head)
        self.drafter.sample_block(self.head.view(1, self.cap, -1), self.pending, out=self.draft)
        self.model.forward(self.verify, self.cache, self.tap, advance=False, logits_out=self.v_logits,
                           fused_out=self.v_fused)
        ops.accept_greedy(self.v_logits.view(1, self.cap + 1, -1), self.draft, seq_lens=self.cache.seq_lens,
                          tt=self.tt, n_out=self.n, token_out=self.token)
        self.drafter.update_context(self.v_fused, 0, self.dcache, n_valid=self.n)

    def run(self, use_graph: bool):
        if use_graph and self.graph is None and self.uses >= 1:
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.body()
        if use_graph and self.graph is not None:
            self.graph.replay()
        else:
            self.body()
        self.uses += 1
        o = self.out.tolist()                                          # the round's one host sync
        n, token, draft = o[0], o[1], o[2:]
        self.cache.note_lengths([self.cache.lengths[0] + n + 1])
        self.dcache.note_lengths([self.dcache.lengths[0] + n + 1])
        return n, token, draft


def speculative_generate(target_model, tokenizer, drafter, prompt: str = "", *, prompt_ids=None, cache=None,
                         ctx_caches=None, reuse_len: int = 0, max_new_tokens: int = 128,
                         confidence_threshold: float = 0.0, max_draft_tokens=2, cap_controller=None,
                         lookup_drafts: bool = True, lookup_max_draft: int = 6, temperature: float = 0.0,
                         top_p: float = 1.0, top_k: int = 0, presence_penalty: float = 0.0,
                         frequency_penalty: float = 0.0, logprobs=None, seed=None, apply_chat_template: bool = True,
                         stop=None, on_text=None, verbose: bool = False, use_graph: bool = True,
                         max_ctx: int | None = None) -> GenResult:
    """Speculative decoding with a DSpark drafter, batch 1 (src/mlx_dspark/generate.py:691-978).

    Greedy (temperature 0): Markov-argmax draft, exact argmax-match verify; the output is the
    target's greedy stream. temperature > 0: speculative sampling (accept with min(1, p/q),
    residual resample, bonus from the target), exact wrt truncate(softmax(target / T)).
    max_draft_tokens caps the drafted-and-verified positions per round (None = the whole
    block); confidence_threshold > 0 truncates the draft with the confidence head's
    cumulative survival; lookup_drafts verifies an n-gram continuation of an earlier
    occurrence instead of drafting when one exists. The default greedy round (no penalties,
    no confidence truncation) runs on the device end to end, graph-replayed, with one host
    sync per round."""
    cfg = drafter.config
    tap = list(cfg.target_layer_ids)
    k = int(cfg.block_size)
    cap_ceiling = k if max_draft_tokens is None else max(1, min(int(max_draft_tokens), k))
    eos_ids = eos_token_ids(tokenizer)
    ids = prompt_ids if prompt_ids is not None else encode_prompt(tokenizer, prompt, apply_chat_template)
    model = target_model.model
    V = model.args.vocab_size
    need = len(ids) + max_new_tokens + 2 * (k + max(lookup_max_draft, k)) + 8
    if cache is None:
        cache = target_model.make_cache(max_ctx=max(max_ctx or 0, need))
        ctx_caches = drafter.make_ctx_cache(max_ctx=max(max_ctx or 0, need))
        reuse_len = 0
    elif ctx_caches is None:
        raise ValueError("a reused target cache needs its drafter ctx_caches")
    st = TextStream(tokenizer, eos_ids, on_text, stop)
    s64 = _seed64(seed)
    t0 = time.time()

    suffix = ids[reuse_len:] if reuse_len else ids
    if reuse_len and (cache.lengths[0] != reuse_len or ctx_caches.lengths[0] != reuse_len):
        raise ValueError(f"reused caches hold {cache.lengths[0]} / {ctx_caches.lengths[0]} tokens, "
                         f"reuse_len={reuse_len}")

    def feed(fused, pos):
        drafter.update_context(fused, pos, ctx_caches)

    logits, _ = model.prefill(suffix, cache, tap, on_chunk=feed)
    pending = _pick(logits[0, -1], temperature, top_p, top_k, s64, 0xFFFFFFFF)
    pen = _Penalizer(presence_penalty, frequency_penalty)
    pen.add([pending])
    lp_list: list | None = [] if logprobs is not None else None
    if lp_list is not None:                                  # the first token came from the prefill row
        lp_list.extend(_logprobs_for_block(logits[0, -1:], [pending], logprobs))
    index = None
    if lookup_drafts:
        from .lookup import NGramIndex
        index = NGramIndex(min_n=4, max_n=5, max_draft=max(1, lookup_max_draft))
        index.extend(list(ids) + [pending])

    out_ids = [pending]
    accept_lengths: list = []
    target_forwards = 1
    lookup_rounds = 0
    rounds: dict = {}
    mask_id = int(cfg.mask_token_id)
    dev = model.device
    st.feed(out_ids)
    r = 0
    while len(out_ids) < max_new_tokens and pending not in eos_ids and not st.closed:
        lk = index.propose() if index is not None else []
        cap = cap_ceiling if cap_controller is None else max(1, min(int(cap_controller.cap), cap_ceiling))
        width = 1 + (len(lk) if lk else cap)
        if cache.lengths[0] + width > cache.max_ctx or ctx_caches.lengths[0] + width + k > ctx_caches.max_ctx:
            break
        use_conf = confidence_threshold > 0.0 and drafter.confidence_head is not None
        fast = not lk and temperature <= 0.0 and not use_conf and not pen.active
        if fast:
            rnd = rounds.get(cap)
            if rnd is None:
                rnd = rounds[cap] = _DSparkRound(target_model, drafter, cache, ctx_caches, cap)
            rnd.pending.fill_(pending)
            n, tok, draft = rnd.run(use_graph)
            raw = rnd.v_logits                                # static buffer, unpenalised
        else:
            q_logits = None
            if lk:
                lookup_rounds += 1
                draft = list(lk)
            else:
                block = torch.tensor([[pending] + [mask_id] * (k - 1)], dtype=torch.int32, device=dev)
                hb = drafter.block_hidden(block, ctx_caches)[:cap]
                base = blockdraft.head_rows(drafter, hb, drafter.lm_head).view(1, cap, -1)
                if temperature > 0.0:
                    d_t, q_logits = drafter.sample_block_probs(base[0], pending, temperature, top_p, top_k,
                                                               seed=s64, offset=r)
                else:
                    d_t = drafter.sample_block(base[0], pending)
                draft = [int(x) for x in d_t.tolist()]
                if use_conf:
                    normed = ops.pack(hb, drafter.norm, cfg.rms_norm_eps).unpack()
                    conf = torch.sigmoid(drafter.confidence_logits(normed, [pending] + draft[:-1])).tolist()
                    surv, keep = 1.0, 0
                    for i, c in enumerate(conf):
                        surv *= c
                        if surv < confidence_threshold:
                            break
                        keep = i + 1
                    draft = draft[:max(keep, 1)]
            L = len(draft)
            vids = torch.tensor([[pending] + draft], dtype=torch.int32, device=dev)
            v_logits, v_fused = model.forward(vids, cache, tap, advance=False)
            raw = v_logits[0]
            v_logits = pen.apply(raw.clone() if pen.active and lp_list is not None else raw, draft)
            n_t = torch.zeros(1, dtype=torch.int32, device=dev)
            tok_t = torch.zeros(1, dtype=torch.int32, device=dev)
            if temperature > 0.0:
                ql = None if lk else q_logits[:L].reshape(1, L, V)
                ops.accept_sample(v_logits.view(1, L + 1, V), ql, torch.tensor([draft], dtype=torch.int32, device=dev),
                                  temperature, top_p, top_k, q_mul_inv_t=True, seed=s64, offset=r,
                                  seq_lens=cache.seq_lens, n_out=n_t, token_out=tok_t)
            else:
                ops.accept_greedy(v_logits.view(1, L + 1, V), torch.tensor([draft], dtype=torch.int32, device=dev),
                                  seq_lens=cache.seq_lens, n_out=n_t, token_out=tok_t)
            drafter.update_context(v_fused[0], 0, ctx_caches, n_valid=n_t)
            n, tok = int(n_t.item()), int(tok_t.item())
            cache.note_lengths([cache.lengths[0] + n + 1])
            ctx_caches.note_lengths([ctx_caches.lengths[0] + n + 1])
        r += 1
        committed = draft[:n] + [tok]
        target_forwards += 1
        accept_lengths.append(len(committed))
        if cap_controller is not None and not lk:
            cap_controller.update(n, len(draft))
        appended = []
        for t in committed:
            out_ids.append(t)
            appended.append(t)
            if t in eos_ids:
                break
        pen.add(appended)
        if lp_list is not None and appended:                  # raw rows at the committed positions
            lp_list.extend(_logprobs_for_block(raw[:len(appended)], appended, logprobs))
        if index is not None:
            index.extend(appended)
        pending = out_ids[-1]
        st.feed(out_ids)
        if verbose:
            print(f"  round {len(accept_lengths):3d}: {'lookup' if lk else 'drafter'} drafted {len(draft)}, "
                  f"accepted {n}, committed {len(committed)}")
    st.close()
    secs = time.time() - t0
    return GenResult(text=st.result_text(out_ids), token_ids=out_ids, num_tokens=len(out_ids),
                     num_rounds=len(accept_lengths), accept_lengths=accept_lengths, target_forwards=target_forwards,
                     seconds=secs, finish_reason=st.finish_reason(out_ids, max_new_tokens, pending),
                     lookup_rounds=lookup_rounds, logprobs=lp_list)
