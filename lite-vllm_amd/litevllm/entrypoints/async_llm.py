"""AsyncLLM: streaming generation on top of LLMEngine.

Public API of the reference's AsyncLLM (entrypoints/async_llm.py:25-126):
``initialize``, ``add_request``, ``stream`` (text deltas), ``generate``,
``abort``, ``has_unfinished``.

Design: one engine thread owns the LLMEngine for its whole life.  The
asyncio side never touches engine state; it posts commands (add, abort,
stop) to the thread's inbox, and the thread applies them between two
``LLMEngine.step`` calls, so the scheduler and the block manager only ever
change on that thread (an abort can never land between a step's schedule
and its packing).  The thread hands each step's outputs back to the event
loop with ``call_soon_threadsafe``; every request has its own
``asyncio.Queue`` of deltas closed by an end marker.  If a step raises,
the error is delivered to every open stream (each ``stream`` raises it)
and later requests are refused.  A consumer that stops reading a stream
early aborts its request, which frees its KV blocks.  ``shutdown`` ends
every stream still open (each raises ``RuntimeError``), including requests
posted after it, and later requests are refused.
"""

from __future__ import annotations

import asyncio
import threading
import uuid
from collections import deque
from typing import AsyncIterator, Optional

from litevllm.config import EngineConfig, SamplingParams
from litevllm.engine.llm_engine import LLMEngine

_END = object()          # end of a stream


class _Failed:
    """A stream item carrying the engine thread's exception."""

    def __init__(self, exc: BaseException) -> None:
        self.exc = exc


class AsyncLLM:
    def __init__(self, engine_config: EngineConfig) -> None:
        self.config = engine_config
        self._engine: Optional[LLMEngine] = None
        self._loop: Optional[asyncio.AbstractEventLoop] = None
        self._streams: dict[str, asyncio.Queue] = {}
        self._inbox: deque = deque()               # (command, payload), loop -> engine thread
        self._wake = threading.Condition()
        self._thread: Optional[threading.Thread] = None
        self._error: Optional[BaseException] = None
        self._closed = False                       # shutdown() was called

    # -- lifecycle ---------------------------------------------------------
    async def initialize(self) -> None:
        """Load the model and start the engine thread."""
        self._loop = asyncio.get_running_loop()
        engine = LLMEngine(self.config)
        engine.stream_text = True
        await self._loop.run_in_executor(None, engine.initialize)
        self._engine = engine
        self._thread = threading.Thread(target=self._run_engine, name="litevllm-engine",
                                        daemon=True)
        self._thread.start()

    async def shutdown(self) -> None:
        """Stop the engine thread.  Unfinished requests are dropped: their
        streams raise ``RuntimeError`` instead of waiting forever."""
        self._closed = True
        if self._thread is not None:
            self._post("stop", None)
            await self._loop.run_in_executor(None, self._thread.join)
            self._thread = None

    # -- requests ------------------------------------------------------------
    async def add_request(self, prompt: Optional[str], sampling_params: SamplingParams,
                          request_id: Optional[str] = None,
                          prompt_token_ids: Optional[list[int]] = None) -> str:
        if self._closed:
            raise RuntimeError("AsyncLLM is shut down")
        if self._thread is None:
            raise RuntimeError("AsyncLLM is not initialized (await initialize() first)")
        if self._error is not None:
            raise RuntimeError("the engine thread failed") from self._error
        if request_id is None:
            request_id = str(uuid.uuid4())
        if request_id in self._streams:
            raise ValueError(f"request {request_id!r} is already running")
        self._streams[request_id] = asyncio.Queue()
        self._post("add", (request_id, prompt, sampling_params, prompt_token_ids))
        return request_id

    async def stream(self, prompt: Optional[str], sampling_params: Optional[SamplingParams] = None,
                     request_id: Optional[str] = None,
                     prompt_token_ids: Optional[list[int]] = None) -> AsyncIterator[str]:
        """Yield the request's output text as it is produced, one delta per
        step that added text."""
        if sampling_params is None:
            sampling_params = SamplingParams(temperature=0.0, max_tokens=256)
        request_id = await self.add_request(prompt, sampling_params, request_id, prompt_token_ids)
        queue = self._streams[request_id]
        done = False
        try:
            while True:
                item = await queue.get()
                if item is _END:
                    done = True
                    return
                if isinstance(item, _Failed):
                    done = True
                    raise RuntimeError(f"request {request_id} failed in the engine") from item.exc
                yield item
        finally:
            self._streams.pop(request_id, None)
            if not done and self._thread is not None:
                self._post("abort", request_id)     # the reader went away

    async def generate(self, prompt: str, sampling_params: Optional[SamplingParams] = None) -> str:
        return "".join([d async for d in self.stream(prompt, sampling_params)])

    async def abort(self, request_id: str) -> None:
        """Stop a request; its stream ends once the engine thread applied it."""
        if self._thread is not None:
            self._post("abort", request_id)

    @property
    def has_unfinished(self) -> bool:
        eng = self._engine
        with self._wake:
            pending = bool(self._inbox)
        return eng is not None and (pending or eng.has_unfinished())

    # -- engine thread -------------------------------------------------------
    def _post(self, command: str, payload) -> None:
        with self._wake:
            self._inbox.append((command, payload))
            self._wake.notify()

    def _to_loop(self, fn, *args) -> None:
        try:
            self._loop.call_soon_threadsafe(fn, *args)
        except RuntimeError:      # the event loop is closed: nobody is listening
            pass

    def _run_engine(self) -> None:
        eng = self._engine
        while True:
            with self._wake:
                while not self._inbox and not eng.has_unfinished():
                    self._wake.wait()
                commands = list(self._inbox)
                self._inbox.clear()
            for command, payload in commands:
                if command == "stop":
                    # every stream still open ends now, also those whose
                    # "add" came after the stop (never applied: the engine
                    # is not stepped again)
                    self._to_loop(self._fail_all, RuntimeError("AsyncLLM shut down"))
                    return
                if command == "add":
                    rid, prompt, params, ids = payload
                    try:
                        eng.add_request(prompt, params, rid, prompt_token_ids=ids)
                    except Exception as exc:       # bad request: only its stream fails
                        self._to_loop(self._deliver, rid, _Failed(exc))
                elif command == "abort":
                    eng.scheduler.abort_request(payload)
                    self._to_loop(self._deliver, payload, _END)
            if not eng.has_unfinished():
                continue
            try:
                outputs = eng.step()
            except BaseException as exc:           # the engine is unusable now
                self._error = exc
                self._to_loop(self._fail_all, exc)
                return
            if outputs:
                self._to_loop(self._dispatch, outputs)

    # -- event-loop side -----------------------------------------------------
    def _deliver(self, request_id: str, item) -> None:
        queue = self._streams.get(request_id)
        if queue is not None:
            queue.put_nowait(item)

    def _dispatch(self, outputs) -> None:
        for out in outputs:
            queue = self._streams.get(out.request_id)
            if queue is None:
                continue
            if out.delta_text:
                queue.put_nowait(out.delta_text)
            if out.finished:
                queue.put_nowait(_END)

    def _fail_all(self, exc: BaseException) -> None:
        for queue in self._streams.values():
            queue.put_nowait(_Failed(exc))
