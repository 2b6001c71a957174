"""AsyncLLM — streaming generation (reference entrypoints/async_llm.py:
25-126): engine steps run on an executor thread, one asyncio.Queue per
request, text deltas streamed, a None sentinel ends a stream."""

from __future__ import annotations

import asyncio
import uuid
from typing import AsyncIterator, Optional

from litevllm.config import EngineConfig, SamplingParams
from litevllm.engine.llm_engine import LLMEngine


class AsyncLLM:
    def __init__(self, engine_config: EngineConfig) -> None:
        self.config = engine_config
        self._engine: Optional[LLMEngine] = None
        self._request_streams: dict[str, asyncio.Queue] = {}
        self._step_task: Optional[asyncio.Task] = None
        self._running = False

    async def initialize(self) -> None:
        self._engine = LLMEngine(self.config)
        self._engine.stream_text = True
        await asyncio.get_running_loop().run_in_executor(None, self._engine.initialize)

    async def add_request(self, prompt: Optional[str], sampling_params: SamplingParams,
                          request_id: Optional[str] = None,
                          prompt_token_ids: Optional[list[int]] = None) -> str:
        if request_id is None:
            request_id = str(uuid.uuid4())
        self._request_streams[request_id] = asyncio.Queue()
        self._engine.add_request(prompt, sampling_params, request_id, prompt_token_ids)
        self._ensure_step_loop()
        return request_id

    async def stream(self, prompt: Optional[str], sampling_params: Optional[SamplingParams] = None,
                     request_id: Optional[str] = None,
                     prompt_token_ids: Optional[list[int]] = None) -> AsyncIterator[str]:
        if sampling_params is None:
            sampling_params = SamplingParams(temperature=0.0, max_tokens=256)
        request_id = await self.add_request(prompt, sampling_params, request_id, prompt_token_ids)
        queue = self._request_streams[request_id]
        try:
            while True:
                item = await queue.get()
                if item is None:
                    break
                yield item
        finally:
            self._request_streams.pop(request_id, None)

    async def generate(self, prompt: str, sampling_params: Optional[SamplingParams] = None) -> str:
        return "".join([d async for d in self.stream(prompt, sampling_params)])

    def _ensure_step_loop(self) -> None:
        if self._running:
            return
        self._running = True
        self._step_task = asyncio.ensure_future(self._step_loop())

    async def _step_loop(self) -> None:
        loop = asyncio.get_running_loop()
        try:
            while self._engine.has_unfinished():
                outputs = await loop.run_in_executor(None, self._engine.step)
                for out in outputs:
                    queue = self._request_streams.get(out.request_id)
                    if queue is None:
                        continue
                    if out.delta_text:
                        await queue.put(out.delta_text)
                    if out.finished:
                        await queue.put(None)
                await asyncio.sleep(0)
        finally:
            self._running = False
            self._step_task = None

    async def abort(self, request_id: str) -> None:
        self._engine.scheduler.abort_request(request_id)
        queue = self._request_streams.pop(request_id, None)
        if queue is not None:
            await queue.put(None)

    @property
    def has_unfinished(self) -> bool:
        return self._engine is not None and self._engine.has_unfinished()
