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
