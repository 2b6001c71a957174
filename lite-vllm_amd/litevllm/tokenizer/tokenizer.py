"""Tokenizer wrapper with the reference's interface (tokenizer/tokenizer.py:
11-93): encode / decode / eos_token_id (falls back to 0 when the tokenizer
has none), one cached instance per (name, revision)."""

from __future__ import annotations

import threading
from functools import lru_cache
from typing import Optional


class TokenizerGroup:
    def __init__(self, name: str, trust_remote_code: bool = True,
                 revision: Optional[str] = None) -> None:
        from transformers import AutoTokenizer
        self._tok = AutoTokenizer.from_pretrained(name, trust_remote_code=trust_remote_code,
                                                  revision=revision)
        self._lock = threading.Lock()

    @classmethod
    def wrap(cls, tokenizer) -> "TokenizerGroup":
        """A group around an already constructed Hugging Face tokenizer."""
        g = cls.__new__(cls)
        g._tok = tokenizer
        g._lock = threading.Lock()
        return g

    def encode(self, text: str) -> list[int]:
        with self._lock:
            return self._tok.encode(text)

    def decode(self, ids: list[int], skip_special_tokens: bool = True) -> str:
        with self._lock:
            return self._tok.decode(ids, skip_special_tokens=skip_special_tokens)

    @property
    def eos_token_id(self) -> int:
        eos = self._tok.eos_token_id
        return 0 if eos is None else eos

    @property
    def vocab_size(self) -> int:
        return len(self._tok)


@lru_cache(maxsize=8)
def get_tokenizer(name: str, trust_remote_code: bool = True,
                  revision: Optional[str] = None) -> TokenizerGroup:
    return TokenizerGroup(name, trust_remote_code, revision)
