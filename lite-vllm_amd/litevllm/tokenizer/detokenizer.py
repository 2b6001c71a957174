"""Incremental detokenization: the text of a growing id list in O(window)
per appended token instead of re-decoding the whole output every step (the
reference decodes all output ids per step for the streamed delta,
engine/llm_engine.py:151-158, and again for stop strings, 213-219).

State per stream: ``text`` (what has been emitted), ``prefix_offset`` and
``read_offset``.  Each update decodes ``ids[prefix_offset:]`` and
``ids[prefix_offset:read_offset]`` and emits the difference.  Decoding with a
few already-emitted tokens in front keeps the context-dependent parts of
decoding (a word piece's leading space, clean-up of spaces before
punctuation) the same as in a full decode.  A window whose text ends in
U+FFFD is an incomplete UTF-8 sequence (a character split over byte-level
tokens): nothing is emitted until the next token completes it.
"""

from __future__ import annotations

from typing import Protocol, Sequence

# Tokens kept in front of the new ones.  Six covers the context any
# Hugging Face decoder consults for the join of two tokens.
_CONTEXT = 6


class _Decoder(Protocol):
    def decode(self, ids: list[int], skip_special_tokens: bool = True) -> str: ...


class IncrementalDetokenizer:
    __slots__ = ("skip_special_tokens", "text", "prefix_offset", "read_offset")

    def __init__(self, skip_special_tokens: bool) -> None:
        self.skip_special_tokens = skip_special_tokens
        self.text = ""
        self.prefix_offset = 0
        self.read_offset = 0

    def update(self, tokenizer: _Decoder, ids: Sequence[int]) -> str:
        """Append the text of ids[read_offset:] and return it (the delta;
        empty while a multi-byte character is still incomplete)."""
        n = len(ids)
        if n <= self.read_offset:
            return ""
        skip = self.skip_special_tokens
        window = list(ids[self.prefix_offset:n])
        known = tokenizer.decode(window[:self.read_offset - self.prefix_offset],
                                 skip_special_tokens=skip) if self.read_offset > self.prefix_offset \
            else ""
        full = tokenizer.decode(window, skip_special_tokens=skip)
        if full.endswith("\ufffd"):
            return ""   # incomplete character: wait for the token that ends it
        # text emitted earlier is never taken back; the final output of a
        # request is one full decode, so a clean-up across the join of two
        # windows cannot change what the request returns
        delta = full[len(known):]
        self.text += delta
        self.read_offset = n
        self.prefix_offset = max(self.prefix_offset, n - _CONTEXT)
        return delta
