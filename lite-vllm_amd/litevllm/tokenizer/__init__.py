from .detokenizer import IncrementalDetokenizer
from .tokenizer import TokenizerGroup, get_tokenizer

__all__ = ["IncrementalDetokenizer", "TokenizerGroup", "get_tokenizer"]
