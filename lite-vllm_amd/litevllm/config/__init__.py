from .config import (CacheConfig, EngineConfig, ModelConfig, SamplingParams, SchedulerConfig)

__all__ = ["CacheConfig", "EngineConfig", "ModelConfig", "SamplingParams", "SchedulerConfig"]
