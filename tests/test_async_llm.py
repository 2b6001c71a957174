"""AsyncLLM's concurrency on the CPU, with a scripted stand-in for
LLMEngine (same methods AsyncLLM calls): streams, abort, a reader that
leaves early, a failing request and a failing engine step.  The engine
thread is the only one that touches engine state."""

from __future__ import annotations

import asyncio
import threading

import pytest

from litevllm.config import EngineConfig, ModelConfig, SamplingParams
from litevllm.engine.sequence import SequenceGroupOutput
from litevllm.entrypoints import async_llm as mod


class FakeScheduler:
    def __init__(self, eng):
        self.eng = eng

    def abort_request(self, rid):
        self.eng.check_thread()
        self.eng.active.pop(rid, None)
        self.eng.aborted.append(rid)


class FakeEngine:
    """One token per step per active request; step number `fail_at` raises."""
    fail_at = None

    def __init__(self, config):
        self.active: dict[str, list] = {}
        self.aborted: list[str] = []
        self.scheduler = FakeScheduler(self)
        self.steps = 0
        self.thread = None
        self.stream_text = False

    def check_thread(self):
        if self.thread is None:
            self.thread = threading.get_ident()
        assert threading.get_ident() == self.thread, "engine state touched from two threads"

    def initialize(self):
        pass

    def add_request(self, prompt, params, rid, prompt_token_ids=None):
        self.check_thread()
        if not prompt_token_ids:
            raise ValueError("empty prompt")
        self.active[rid] = [0, params.max_tokens]

    def has_unfinished(self):
        return bool(self.active)

    def step(self):
        self.check_thread()
        self.steps += 1
        if self.fail_at is not None and self.steps == self.fail_at:
            raise RuntimeError("device lost")
        outs = []
        for rid, st in list(self.active.items()):
            st[0] += 1
            done = st[0] >= st[1]
            outs.append(SequenceGroupOutput(rid, "", [], [], "", "length" if done else "running",
                                            delta_text=f"t{st[0]}", finished=done))
            if done:
                del self.active[rid]
        return outs


@pytest.fixture
def fake(monkeypatch):
    FakeEngine.fail_at = None
    monkeypatch.setattr(mod, "LLMEngine", FakeEngine)
    return FakeEngine


def _cfg():
    return EngineConfig(model_config=ModelConfig("fake"))


def _run(coro):
    return asyncio.run(asyncio.wait_for(coro, 20))


def test_streams_run_concurrently_and_finish(fake):
    async def main():
        llm = mod.AsyncLLM(_cfg())
        await llm.initialize()

        async def collect(n):
            return [d async for d in llm.stream(None, SamplingParams(max_tokens=n),
                                                prompt_token_ids=[1])]
        a, b = await asyncio.gather(collect(3), collect(5))
        assert a == ["t1", "t2", "t3"] and b == ["t1", "t2", "t3", "t4", "t5"]
        assert not llm.has_unfinished
        await llm.shutdown()
    _run(main())


def test_abort_ends_the_stream_on_the_engine_thread(fake):
    async def main():
        llm = mod.AsyncLLM(_cfg())
        await llm.initialize()
        got = []
        async for d in llm.stream(None, SamplingParams(max_tokens=1000), request_id="r",
                                  prompt_token_ids=[1]):
            got.append(d)
            if len(got) == 3:
                await llm.abort("r")
        assert 3 <= len(got) < 1000
        assert llm._engine.aborted == ["r"] and not llm._engine.active
        await llm.shutdown()
    _run(main())


def test_reader_leaving_early_aborts_its_request(fake):
    async def main():
        llm = mod.AsyncLLM(_cfg())
        await llm.initialize()
        async for d in llm.stream(None, SamplingParams(max_tokens=1000), request_id="x",
                                  prompt_token_ids=[1]):
            break
        for _ in range(200):
            if "x" in llm._engine.aborted:
                break
            await asyncio.sleep(0.01)
        assert "x" in llm._engine.aborted and not llm._engine.active
        await llm.shutdown()
    _run(main())


def test_bad_request_fails_only_its_stream(fake):
    async def main():
        llm = mod.AsyncLLM(_cfg())
        await llm.initialize()

        async def bad():
            return [d async for d in llm.stream(None, SamplingParams(max_tokens=2),
                                                prompt_token_ids=[])]
        good = llm.stream(None, SamplingParams(max_tokens=4), prompt_token_ids=[1])
        with pytest.raises(RuntimeError) as e:
            await bad()
        assert isinstance(e.value.__cause__, ValueError)
        assert [d async for d in good] == ["t1", "t2", "t3", "t4"]
        await llm.shutdown()
    _run(main())


def test_failed_step_reaches_every_stream_and_refuses_new_requests(fake):
    fake.fail_at = 3

    async def main():
        llm = mod.AsyncLLM(_cfg())
        await llm.initialize()

        async def collect(n):
            return [d async for d in llm.stream(None, SamplingParams(max_tokens=n),
                                                prompt_token_ids=[1])]
        res = await asyncio.gather(collect(50), collect(60), return_exceptions=True)
        for r in res:
            assert isinstance(r, RuntimeError) and "device lost" in str(r.__cause__)
        with pytest.raises(RuntimeError, match="engine thread failed"):
            await llm.add_request(None, SamplingParams(), prompt_token_ids=[1])
    _run(main())


def test_shutdown_ends_open_streams_and_refuses_new_requests(fake):
    async def main():
        llm = mod.AsyncLLM(_cfg())
        await llm.initialize()
        got = []

        async def collect(rid, n):
            async for d in llm.stream(None, SamplingParams(max_tokens=n), request_id=rid,
                                      prompt_token_ids=[1]):
                got.append((rid, d))
        long = asyncio.ensure_future(collect("long", 10**9))
        while len(got) < 2:
            await asyncio.sleep(0.001)
        # posted right before the stop: applied or not, its stream must end
        late = asyncio.ensure_future(collect("late", 10**9))
        await asyncio.sleep(0)
        await llm.shutdown()
        for task in (long, late):
            with pytest.raises(RuntimeError) as e:
                await task
            assert "shut down" in str(e.value.__cause__)
        with pytest.raises(RuntimeError, match="shut down"):
            await llm.add_request(None, SamplingParams(), prompt_token_ids=[1])
    _run(main())
