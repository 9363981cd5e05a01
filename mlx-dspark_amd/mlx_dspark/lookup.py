"""Prompt-lookup (n-gram) drafting index (drop-in for NGramIndex, src/mlx_dspark/lookup.py:44-89).

For every n-gram of length min_n..max_n in the growing token sequence the index keeps the
continuation positions of its two most recent occurrences; a query for the current suffix
skips the suffix's own occurrence and proposes the continuation of the latest earlier one,
longest n first. The speculative loop verifies such a draft instead of running the drafter
(it only changes which tokens are verified, never the output).
"""

from __future__ import annotations


class NGramIndex:
    def __init__(self, min_n: int = 3, max_n: int = 4, max_draft: int = 6):
        self.min_n = max(1, int(min_n))
        self.max_n = max(self.min_n, int(max_n))
        self.max_draft = max(1, int(max_draft))
        self.tokens: list[int] = []
        self._pos: dict[tuple, tuple] = {}   # ngram -> (earlier continuation start, latest)

    def extend(self, new_tokens) -> None:
        for t in new_tokens:
            self.tokens.append(int(t))
            end = len(self.tokens)
            for n in range(self.min_n, min(self.max_n, end) + 1):
                key = tuple(self.tokens[end - n:end])
                old = self._pos.get(key)
                self._pos[key] = (None if old is None else old[1], end)

    def propose(self) -> list[int]:
        end = len(self.tokens)
        for n in range(min(self.max_n, end), self.min_n - 1, -1):
            hit = self._pos.get(tuple(self.tokens[end - n:end]))
            if hit is None:
                continue
            start = hit[0] if hit[1] == end else hit[1]
            if start is None:
                continue
            draft = self.tokens[start:start + self.max_draft]
            if draft:
                return draft
        return []


def lookup_generate(target_model, tokenizer, prompt: str = "", *, prompt_ids=None, cache=None, reuse_len: int = 0,
                    max_new_tokens: int = 128, max_draft_tokens: int = 6, ngram_min: int = 3, ngram_max: int = 4,
                    temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0, seed=None,
                    apply_chat_template: bool = True, stop=None, on_text=None):
    """Prompt-lookup speculative decoding, batch 1, no drafter model (src/mlx_dspark/lookup.py:92-202).

    Each round verifies the n-gram continuation the index proposes ([pending] + draft in one
    target forward) and accepts on the device: greedy is the argmax-match prefix plus one
    token (the target's greedy stream), temperature > 0 is speculative sampling with a
    point-mass proposal at each drafted token (an exact sample of the truncated target
    distribution). With no proposal the round is a plain one-token step. cache / reuse_len
    reuse a prefix exactly as in greedy_generate."""
    import time

    import torch

    from . import ops
    from .generate import GenResult, _pick, _seed64
    from .textstream import TextStream, encode_prompt, eos_token_ids
    eos_ids = eos_token_ids(tokenizer)
    ids = prompt_ids if prompt_ids is not None else encode_prompt(tokenizer, prompt, apply_chat_template)
    model = target_model.model
    if cache is None:
        cache = target_model.make_cache(max_ctx=len(ids) + max_new_tokens + max_draft_tokens + 8)
        reuse_len = 0
    elif reuse_len and cache.lengths[0] != reuse_len:
        raise ValueError(f"reused cache holds {cache.lengths[0]} tokens, reuse_len={reuse_len}")
    st = TextStream(tokenizer, eos_ids, on_text, stop)
    s64 = _seed64(seed)
    index = NGramIndex(min_n=ngram_min, max_n=ngram_max, max_draft=max(1, max_draft_tokens))
    index.extend(ids)
    dev = model.device
    V = model.args.vocab_size

    t0 = time.time()
    logits, _ = model.prefill(ids[reuse_len:] if reuse_len else ids, cache)
    pending = _pick(logits[0, -1], temperature, top_p, top_k, s64, 0xFFFFFFFF)
    out_ids = [pending]
    index.extend([pending])
    accept_lengths: list = []
    target_forwards = 1
    n_t = torch.zeros(1, dtype=torch.int32, device=dev)
    tok_t = torch.zeros(1, dtype=torch.int32, device=dev)
    r = lookup_rounds = 0
    st.feed(out_ids)
    while len(out_ids) < max_new_tokens and pending not in eos_ids and not st.closed:
        draft = index.propose()
        if cache.lengths[0] + 1 + len(draft) > cache.max_ctx:
            break
        if not draft:
            lg, _ = model.forward(torch.tensor([[pending]], dtype=torch.int32, device=dev), cache, None)
            committed = [_pick(lg[0, -1], temperature, top_p, top_k, s64, r)]
        else:
            lookup_rounds += 1
            L = len(draft)
            vids = torch.tensor([[pending] + draft], dtype=torch.int32, device=dev)
            d_t = vids[:, 1:].contiguous()
            v_logits, _ = model.forward(vids, cache, None, advance=False)
            if temperature > 0.0:
                ops.accept_sample(v_logits.view(1, L + 1, V), None, d_t, temperature, top_p, top_k, seed=s64,
                                  offset=r, seq_lens=cache.seq_lens, n_out=n_t, token_out=tok_t)
            else:
                ops.accept_greedy(v_logits.view(1, L + 1, V), d_t, seq_lens=cache.seq_lens, n_out=n_t,
                                  token_out=tok_t)
            n, tok = int(n_t.item()), int(tok_t.item())
            cache.note_lengths([cache.lengths[0] + n + 1])
            committed = draft[:n] + [tok]
        r += 1
        target_forwards += 1
        accept_lengths.append(len(committed))
        appended = []
        for t in committed:
            out_ids.append(t)
            appended.append(t)
            if t in eos_ids:
                break
        index.extend(appended)
        pending = out_ids[-1]
        st.feed(out_ids)
    st.close()
    secs = time.time() - t0
    return GenResult(text=st.result_text(out_ids), token_ids=out_ids, num_tokens=len(out_ids),
                     num_rounds=len(accept_lengths), accept_lengths=accept_lengths, target_forwards=target_forwards,
                     seconds=secs, finish_reason=st.finish_reason(out_ids, max_new_tokens, pending),
                     lookup_rounds=lookup_rounds)
