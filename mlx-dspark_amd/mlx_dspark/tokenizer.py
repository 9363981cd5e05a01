"""A stand-in tokenizer for synthetic models (no vocabulary files exist offline).

encode() maps UTF-8 bytes to ids, decode() renders each id as "<id>"; the rendering of a
prefix of ids is a prefix of the rendering of the whole, which the incremental streamer
relies on. Synthetic models have no eos token unless one is given."""

from __future__ import annotations


class SyntheticTokenizer:
    chat_template = None

    def __init__(self, vocab_size: int, eos_token_id: int | None = None):
        self.vocab_size = int(vocab_size)
        self.eos_token_id = eos_token_id
        self.unk_token_id = None

    def encode(self, text: str) -> list:
        return [b % self.vocab_size for b in text.encode("utf-8")]

    def decode(self, ids) -> str:
        return "".join(f"<{int(i)}>" for i in ids)
