from .tokenizer import TokenizerGroup, get_tokenizer

__all__ = ["TokenizerGroup", "get_tokenizer"]
