from .base import BaseModelForCausalLM

__all__ = ["BaseModelForCausalLM"]
