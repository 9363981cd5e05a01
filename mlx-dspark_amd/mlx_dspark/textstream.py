"""Host-side text of a completion: prompt encoding, end-of-turn ids, streaming with stop strings.

The observable behaviour follows the reference's text helpers (src/mlx_dspark/generate.py:
69-130 for the tokenizer helpers, :294-370 for streaming, stop strings and the finish reason;
their tests are tests/test_generate_helpers.py:17-142): the completion's text is the decode of
its ids without end-of-turn ids, it ends before the earliest stop string, nothing of a stop
string is ever streamed, and StopStreaming raised from the streaming callback ends generation
at the next round boundary with the text decoded so far.
"""

from __future__ import annotations


class StopStreaming(Exception):
    """Raised from an on_text callback to end generation at the next round boundary with a
    normal (partial) GenResult and consistent caches (src/mlx_dspark/generate.py:231-235)."""


# markers that end a turn in the chat formats the reference's targets use; an id counts only
# when the vocabulary knows the marker (not the unknown-token id)
TURN_END_MARKERS = ("<turn|>", "<end_of_turn>", "<|im_end|>", "<|endoftext|>", "<eos>")


def eos_token_ids(tokenizer) -> set:
    """The ids that end a completion: the tokenizer's eos id(s) and the turn-end markers its
    vocabulary holds."""
    ids: set = set()
    for attr in ("eos_token_ids", "eos_token_id"):
        v = getattr(tokenizer, attr, None)
        if v is None:
            continue
        ids.update([v] if isinstance(v, int) else [int(x) for x in v])
    to_id = getattr(tokenizer, "convert_tokens_to_ids", None)
    if to_id is None:
        return ids
    unk = getattr(tokenizer, "unk_token_id", None)
    for marker in TURN_END_MARKERS:
        try:
            i = to_id(marker)
        except Exception:
            continue
        if isinstance(i, int) and i >= 0 and i != unk:
            ids.add(i)
    return ids


def _id_list(result):
    """Token ids of an apply_chat_template result: a list (or a batch of one list), a mapping or
    object with input_ids, or an encoding with .ids. None when it holds no ids."""
    if hasattr(result, "ids") and not isinstance(result, (list, tuple)):
        return list(result.ids)
    if not isinstance(result, (list, tuple)):
        try:
            result = result["input_ids"]
        except (TypeError, KeyError, IndexError):
            result = getattr(result, "input_ids", None)
        if result is None:
            return None
    result = list(result)
    if result and isinstance(result[0], (list, tuple)):
        result = list(result[0])
    return result


def encode_messages(tokenizer, messages, add_generation_prompt=True, **template_kwargs) -> list:
    """Prompt ids of a chat: the tokenizer's chat template when it has one (without the extra
    keywords if the template rejects them), else the messages' contents joined by newlines."""
    if getattr(tokenizer, "chat_template", None):
        for kw in (template_kwargs, {}):
            try:
                ids = _id_list(tokenizer.apply_chat_template(messages, add_generation_prompt=add_generation_prompt,
                                                             **kw))
            except (TypeError, ValueError):
                continue
            if ids is not None:
                return ids
            break
    return list(tokenizer.encode("\n".join(str(m.get("content", "")) for m in messages)))


def encode_prompt(tokenizer, prompt: str, use_chat: bool = True) -> list:
    """Prompt ids of one user message (as a chat when use_chat and the tokenizer has a template)."""
    if use_chat and getattr(tokenizer, "chat_template", None):
        return encode_messages(tokenizer, [{"role": "user", "content": prompt}])
    return list(tokenizer.encode(prompt))


class TextStream:
    """The text of a completion as it grows round by round, cut at the first stop string and
    streamed to ``on_text``.

    feed(out_ids) takes the completion's ids so far (end-of-turn ids are dropped from the text)
    and re-decodes them. A stop string can only start at or after ``_safe``: before it, no
    position starts a stop string or a proper prefix of one, and appended text cannot change
    that. Each feed searches for stop strings from there, then moves ``_safe`` to the start of
    the longest tail of the text that is a proper prefix of a stop string; everything before it
    can be streamed, while that tail waits for the next round (a stop string that straddles two
    rounds is then found whole, and none of it is streamed). A stop string cuts the text before
    its earliest occurrence and closes the stream; so does StopStreaming from on_text, keeping the
    text decoded so far. close() streams the rest at the end of generation."""

    def __init__(self, tokenizer, eos_ids, on_text=None, stop=None):
        self.tokenizer = tokenizer
        self.eos_ids = eos_ids
        self.on_text = on_text
        self.stops = [s for s in (stop or ()) if s]
        self.live = on_text is not None or bool(self.stops)   # otherwise the text is decoded once, at the end
        self.closed = False
        self.text = ""
        self._kept: list = []       # ids of the text (end-of-turn ids removed)
        self._seen = 0              # how many of out_ids have been taken
        self._safe = 0
        self._sent = 0              # characters handed to on_text

    def _held_from(self, text: str) -> int:
        start = len(text)
        for s in self.stops:
            for k in range(min(len(s) - 1, len(text)), 0, -1):
                if text.endswith(s[:k]):
                    start = min(start, len(text) - k)
                    break
        return start

    def _send(self, end: int) -> None:
        if self.on_text is None or end <= self._sent:
            return
        piece = self.text[self._sent:end]
        self._sent = end
        try:
            self.on_text(piece)
        except StopStreaming:
            self.on_text = None
            self.closed = True

    def feed(self, out_ids) -> None:
        if not self.live or self.closed:
            return
        self._kept += [t for t in out_ids[self._seen:] if t not in self.eos_ids]
        self._seen = len(out_ids)
        text = self.tokenizer.decode(self._kept)
        hits = [i for i in (text.find(s, self._safe) for s in self.stops) if i >= 0]
        if hits:
            self.text = text[:min(hits)]
            self.closed = True
            self._send(len(self.text))
            return
        self.text = text
        self._safe = self._held_from(text)
        self._send(self._safe)

    def close(self) -> None:
        """End of generation: stream what was held back (no stop string can complete now)."""
        if self.live and not self.closed:
            self._send(len(self.text))

    def result_text(self, out_ids) -> str:
        if self.closed:
            return self.text
        return self.tokenizer.decode([t for t in out_ids if t not in self.eos_ids])

    def finish_reason(self, out_ids, max_new_tokens: int, last_tok) -> str:
        """"length" when the token budget ended the completion, "stop" otherwise (an end-of-turn
        id, a stop string, a closed stream)."""
        ended = self.closed or last_tok in self.eos_ids
        return "length" if not ended and len(out_ids) >= max_new_tokens else "stop"
