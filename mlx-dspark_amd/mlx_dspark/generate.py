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

import time
from dataclasses import dataclass

import torch

from . import ops

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


class StopStreaming(Exception):
    """Raised from an on_text callback to end generation at the next round boundary with a
    normal (partial) GenResult and consistent caches (src/mlx_dspark/generate.py:231-235)."""


# ============================================================================ tokenizer helpers
def eos_token_ids(tokenizer) -> set:
    """eos ids plus the usual turn-end markers the tokenizer knows (unknown id excluded)."""
    out: set = set()
    for attr in ("eos_token_ids", "eos_token_id"):
        v = getattr(tokenizer, attr, None)
        if isinstance(v, int):
            out.add(v)
        elif v:
            out.update(int(x) for x in v)
    unk = getattr(tokenizer, "unk_token_id", None)
    conv = getattr(tokenizer, "convert_tokens_to_ids", None)
    if conv is not None:
        for t in ("<turn|>", "<end_of_turn>", "<|im_end|>", "<|endoftext|>", "<eos>"):
            try:
                i = conv(t)
            except Exception:
                continue
            if isinstance(i, int) and i >= 0 and i != unk:
                out.add(i)
    return out


def _flat_ids(r):
    if isinstance(r, (list, tuple)):
        return list(r[0]) if r and isinstance(r[0], (list, tuple)) else list(r)
    ii = r["input_ids"] if hasattr(r, "__contains__") and "input_ids" in r else getattr(r, "input_ids", None)
    if ii is not None:
        ii = list(ii)
        return list(ii[0]) if ii and isinstance(ii[0], (list, tuple)) else ii
    return list(r.ids) if hasattr(r, "ids") else None


def encode_messages(tokenizer, messages, add_generation_prompt=True, **template_kwargs) -> list:
    if getattr(tokenizer, "chat_template", None):
        try:
            r = tokenizer.apply_chat_template(messages, add_generation_prompt=add_generation_prompt, **template_kwargs)
        except (TypeError, ValueError):
            r = tokenizer.apply_chat_template(messages, add_generation_prompt=add_generation_prompt)
        ids = _flat_ids(r)
        if ids is not None:
            return ids
    return list(tokenizer.encode("\n".join(str(m.get("content", "")) for m in messages)))


def encode_prompt(tokenizer, prompt: str, use_chat: bool = True) -> list:
    if use_chat and getattr(tokenizer, "chat_template", None):
        return encode_messages(tokenizer, [{"role": "user", "content": prompt}])
    return list(tokenizer.encode(prompt))


class _Streamer:
    """Round-granular text streaming with stop strings (behaviour of the reference's
    _Streamer, src/mlx_dspark/generate.py:294-362): new tokens are decoded incrementally,
    stop strings are searched from max_stop - 1 characters back so one that straddles two
    rounds is found, and emission holds back the last max_stop - 1 characters until they
    are known not to start a stop string. StopStreaming from on_text ends the loop cleanly."""

    def __init__(self, tokenizer, eos_ids, on_text, stop):
        self.tok = tokenizer
        self.eos = eos_ids
        self.on_text = on_text
        self.stop = [s for s in (stop or []) if s]
        self.max_stop = max((len(s) for s in self.stop), default=0)
        self.active = on_text is not None or bool(self.stop)
        self.ids: list = []
        self.n_fed = 0
        self.scan_from = 0
        self.streamed = 0
        self.text = ""
        self.stopped = False

    def update(self, out_ids) -> None:
        if not self.active or self.stopped:
            return
        self.ids.extend(t for t in out_ids[self.n_fed:] if t not in self.eos)
        self.n_fed = len(out_ids)
        self._advance(final=False)

    def flush(self) -> None:
        if self.active and not self.stopped:
            self._advance(final=True)

    def _advance(self, final: bool) -> None:
        text = self.tok.decode(self.ids)
        if self.stop:
            hits = [i for i in (text.find(s, self.scan_from) for s in self.stop) if i != -1]
            if hits:
                text = text[:min(hits)]
                self.stopped = True
            else:
                self.scan_from = max(0, len(text) - (self.max_stop - 1))
        self.text = text
        if self.on_text is None:
            return
        end = len(text)
        if not (self.stopped or final) and self.max_stop > 1:
            end = max(self.streamed, len(text) - (self.max_stop - 1))
        if end > self.streamed:
            try:
                self.on_text(text[self.streamed:end])
            except StopStreaming:
                self.on_text = None
                self.stopped = True
                return
            self.streamed = end


def _finish_reason(out_ids, max_new_tokens, last_tok, eos_ids, streamer) -> str:
    if streamer.stopped or last_tok in eos_ids:
        return "stop"
    return "length" if len(out_ids) >= max_new_tokens else "stop"


def _final_text(tokenizer, st: _Streamer, out_ids, eos_ids) -> str:
    return st.text if st.stopped else tokenizer.decode([t for t in out_ids if t not in eos_ids])


# ============================================================================ sampling helpers
def _pick(logits_row: torch.Tensor, temperature: float, top_p=1.0, top_k=0, seed=0, offset=0xFFFFFFFF) -> int:
    """argmax (T == 0) or a truncated sample of one logits row (one host sync)."""
    tok, _ = ops.sample_rows(logits_row.reshape(1, -1).float(), temperature, top_p, top_k, seed=seed, offset=offset)
    return int(tok.item())


def _seed64(seed) -> int:
    return 0x5EED if seed is None else int(seed) & ((1 << 64) - 1)


# ============================================================================ greedy baseline
def greedy_generate(target_model, tokenizer, prompt: str = "", *, prompt_ids=None, cache=None, reuse_len: int = 0,
                    max_new_tokens: int = 128, temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0,
                    presence_penalty: float = 0.0, frequency_penalty: float = 0.0, logprobs=None, seed=None,
                    apply_chat_template: bool = True, stop=None, on_text=None) -> GenResult:
    """Plain one-token-per-forward decoding of the target (src/mlx_dspark/generate.py:373-465)."""
    if presence_penalty or frequency_penalty or logprobs is not None:
        raise NotImplementedError("penalties and logprobs are not supported by this engine yet")
    eos_ids = eos_token_ids(tokenizer)
    ids = prompt_ids if prompt_ids is not None else encode_prompt(tokenizer, prompt, apply_chat_template)
    if cache is None:
        cache = target_model.make_cache()
        reuse_len = 0
    st = _Streamer(tokenizer, eos_ids, on_text, stop)
    s64 = _seed64(seed)
    t0 = time.time()
    model = target_model.model
    logits, _ = model.prefill(ids[reuse_len:] if reuse_len else ids, cache)
    nxt = _pick(logits[0, -1], temperature, top_p, top_k, s64, 0)
    out_ids = [nxt]
    st.update(out_ids)
    cur = torch.empty((1, 1), dtype=torch.int32, device=model.device)
    step = 1
    while len(out_ids) < max_new_tokens and nxt not in eos_ids and not st.stopped:
        cur.fill_(nxt)
        lg, _ = model.forward(cur, cache, None)
        nxt = _pick(lg[0, -1], temperature, top_p, top_k, s64, step)
        step += 1
        out_ids.append(nxt)
        st.update(out_ids)
    st.flush()
    secs = time.time() - t0
    return GenResult(text=_final_text(tokenizer, st, out_ids, eos_ids), token_ids=out_ids, num_tokens=len(out_ids),
                     num_rounds=len(out_ids), accept_lengths=[1] * len(out_ids), target_forwards=len(out_ids),
                     seconds=secs, finish_reason=_finish_reason(out_ids, max_new_tokens, nxt, eos_ids, st))


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
        self.pending = torch.zeros(1, dtype=torch.int32, device=dev)
        self.draft = torch.zeros(cap, dtype=torch.int32, device=dev)
        self.verify = torch.zeros((1, cap + 1), dtype=torch.int32, device=dev)
        self.head = torch.empty((cap, V), dtype=torch.float32, device=dev)
        self.v_logits = torch.empty((cap + 1, V), dtype=torch.float32, device=dev)
        self.v_fused = torch.empty((cap + 1, len(self.tap) * H), dtype=torch.bfloat16, device=dev)
        self.n = torch.zeros(1, dtype=torch.int32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tt = torch.zeros((1, cap + 1), dtype=torch.int32, device=dev)
        self.out = torch.zeros(2 + cap, dtype=torch.int32, device=dev)   # [n, token, draft...]
        self.graph = None

    def body(self, round_idx: int = 0) -> None:
        self.block[0, 0:1].copy_(self.pending)
        self.drafter.block_logits(self.block, self.dcache, 1, self.cap, out=self.head)
        if self.T > 0:
            q_probs = torch.empty_like(self.head)
            ops.sample_rows(self.head, self.T, self.top_p, self.top_k, seed=self.seed, offset=round_idx,
                            token_out=self.draft, probs_out=q_probs)
        else:
            ops.sample_rows(self.head, 0.0, token_out=self.draft)
        self.verify[0, 0:1].copy_(self.pending)
        self.verify[0, 1:].copy_(self.draft)
        self.model.forward(self.verify, self.cache, self.tap, advance=False, logits_out=self.v_logits,
                           fused_out=self.v_fused)
        if self.T > 0:
            ops.accept_sample(self.v_logits.view(1, self.cap + 1, -1), self.head.view(1, self.cap, -1),
                              self.draft.view(1, -1), self.T, self.top_p, self.top_k, seed=self.seed,
                              offset=round_idx, seq_lens=self.cache.seq_lens, n_out=self.n, token_out=self.token)
        else:
            ops.accept_greedy(self.v_logits.view(1, self.cap + 1, -1), self.draft.view(1, -1),
                              seq_lens=self.cache.seq_lens, tt=self.tt, n_out=self.n, token_out=self.token)
        self.pending.copy_(self.token)
        self.drafter.ingest(self.v_fused, self.dcache, n_valid=self.n)     # commit [anchor, accepted]
        self.out[0:1].copy_(self.n)
        self.out[1:2].copy_(self.token)
        self.out[2:].copy_(self.draft)

    def run(self, round_idx: int, use_graph: bool):
        if use_graph and self.T == 0:
            if self.graph is None and round_idx >= 1:
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph):
                    self.body()
            if self.graph is not None:
                self.graph.replay()
            else:
                self.body(round_idx)
        else:
            self.body(round_idx)
        o = self.out.tolist()                                         # the round's one host sync
        n, token, draft = o[0], o[1], o[2:]
        self.cache.note_lengths([self.cache.lengths[0] + n + 1])
        self.dcache.note_lengths([self.dcache.lengths[0] + n + 1])
        return n, token, draft


def dflash_generate(target_model, tokenizer, drafter, prompt: str = "", *, prompt_ids=None, max_new_tokens: int = 128,
                    max_draft_tokens=None, cap_controller=None, temperature: float = 0.0, top_p: float = 1.0,
                    top_k: int = 0, apply_chat_template: bool = True, seed=None, stop=None, on_text=None,
                    use_graph: bool = True, max_ctx: int | None = None) -> GenResult:
    """Speculative decoding with a DFlash block-diffusion drafter (src/mlx_dspark/generate.py:468-601)."""
    if getattr(drafter, "embed_tokens", None) is None:
        drafter.bind(target_model.model)
    if cap_controller is not None:
        raise NotImplementedError("cap_controller is not supported by this engine")
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
    st = _Streamer(tokenizer, eos_ids, on_text, stop)
    s64 = _seed64(seed)
    t0 = time.time()

    logits, fused = target_model.model.prefill(ids, cache, tap)
    drafter.ingest(fused, dcache)                                     # whole prompt -> draft context
    pending = _pick(logits[0, -1], temperature, top_p, top_k, s64, 0xFFFFFFFF)
    out_ids = [pending]
    accept_lengths: list = []
    target_forwards = 1
    rnd = _DFlashRound(target_model, drafter, cache, dcache, cap, temperature, top_p, top_k, s64)
    rnd.pending.fill_(pending)
    st.update(out_ids)
    r = 0
    while len(out_ids) < max_new_tokens and pending not in eos_ids and not st.stopped:
        if cache.lengths[0] + cap + 1 > cache.max_ctx:
            break
        n, token, draft = rnd.run(r, use_graph)
        r += 1
        committed = draft[:n] + [token]
        target_forwards += 1
        accept_lengths.append(len(committed))
        for tok in committed:
            out_ids.append(tok)
            if tok in eos_ids:
                break
        pending = out_ids[-1]
        st.update(out_ids)
    st.flush()
    secs = time.time() - t0
    return GenResult(text=_final_text(tokenizer, st, out_ids, eos_ids), token_ids=out_ids, num_tokens=len(out_ids),
                     num_rounds=len(accept_lengths), accept_lengths=accept_lengths, target_forwards=target_forwards,
                     seconds=secs, finish_reason=_finish_reason(out_ids, max_new_tokens, pending, eos_ids, st))
