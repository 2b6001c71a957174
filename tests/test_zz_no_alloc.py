"""lv_sample_noalloc (the sampler entry point that allocates nothing, its
scratch a fixed array in the library's device memory) against lv_sample
with a caller workspace, both called through the C ABI: identical ids on
two calls in a row, the second smaller than the first (the scratch keeps
the first call's contents).  The refusal of requests beyond the fixed
scratch is a host-side check, tested without a GPU in test_capi.py."""

from __future__ import annotations

import pytest
import torch

from litevllm import _hip, workloads

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


_DT = {torch.bfloat16: _hip.LV_BF16, torch.float16: _hip.LV_F16, torch.float32: _hip.LV_F32}


def _both(lib, logits, temp, uni):
    B, V = logits.shape
    stream = torch.cuda.current_stream().cuda_stream
    dt = _DT[logits.dtype]
    ws_bytes = int(lib.lv_sample_workspace_size(B, V))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=logits.device)
    want = torch.full((B,), -1, dtype=torch.int64, device=logits.device)
    got = torch.full((B,), -2, dtype=torch.int64, device=logits.device)
    _hip.check(lib.lv_sample(logits.data_ptr(), B, V, logits.stride(0), temp.data_ptr(),
                             uni.data_ptr(), want.data_ptr(), ws.data_ptr(), ws_bytes, dt,
                             stream), "lv_sample")
    _hip.check(lib.lv_sample_noalloc(logits.data_ptr(), B, V, logits.stride(0), temp.data_ptr(),
                                     uni.data_ptr(), got.data_ptr(), dt, stream),
               "lv_sample_noalloc")
    torch.cuda.synchronize()
    return want.cpu(), got.cpu()


def test_sample_noalloc_matches_lv_sample(device):
    lib = _hip.load()
    # call 1: config 4 ([256, 151936] bf16, half greedy, half temperature)
    _say("lv_sample_noalloc call 1: config4 256 x 151936 bf16")
    sb = workloads.sampler_batch(seed=0)
    want, got = _both(lib, sb.logits.to(device), sb.temperature.to(device), sb.uniform.to(device))
    assert torch.equal(got, want)
    assert torch.equal(got[:128], sb.planted[:128])
    # call 2: smaller (40 rows of a 32000 vocab, fp32, from a strided view),
    # so stale entries of call 1 sit beyond what call 2 writes
    _say("lv_sample_noalloc call 2: 40 x 32000 fp32, strided rows")
    sb2 = workloads.sampler_batch(seed=3, rows=40, vocab=32000, dtype=torch.float32)
    wide = torch.zeros(40, 32768, dtype=torch.float32, device=device)
    wide[:, :32000] = sb2.logits.to(device)
    want2, got2 = _both(lib, wide[:, :32000], sb2.temperature.to(device), sb2.uniform.to(device))
    assert torch.equal(got2, want2)
    assert torch.equal(got2[:20], sb2.planted[:20])


def test_sample_noalloc_allocates_nothing_and_replays_in_a_graph(device):
    """After a warm-up call (the scratch address lookup happens on the first
    call on a device), a call changes neither torch's allocation count nor
    the device's free memory, and the call captured in a HIP graph gives
    lv_sample's ids on every replay, with new logits copied into the
    captured input between replays and eager work in between."""
    lib = _hip.load()
    B, V = 64, 32000
    batches = [workloads.sampler_batch(seed=s, rows=B, vocab=V) for s in (5, 6, 7, 8)]
    logits = batches[0].logits.to(device)
    temp = batches[0].temperature.to(device)
    uni = batches[0].uniform.to(device)
    got = torch.full((B,), -2, dtype=torch.int64, device=device)

    def noalloc():
        _hip.check(lib.lv_sample_noalloc(logits.data_ptr(), B, V, V, temp.data_ptr(),
                                         uni.data_ptr(), got.data_ptr(), _hip.LV_BF16,
                                         torch.cuda.current_stream().cuda_stream),
                   "lv_sample_noalloc")

    _say("lv_sample_noalloc: warm-up, then allocation check")
    noalloc()
    torch.cuda.synchronize()
    alloc0, free0 = torch.cuda.memory_allocated(device), torch.cuda.mem_get_info(device)[0]
    noalloc()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(device) == alloc0
    assert torch.cuda.mem_get_info(device)[0] == free0

    _say("lv_sample_noalloc: captured in a graph, 3 replays")
    g = torch.cuda.CUDAGraph()
    # inference mode, as the engine captures its graphs: capture_begin
    # updates the CUDA generator's state, which an earlier engine run in the
    # same process may have created as an inference tensor
    with torch.inference_mode(), torch.cuda.graph(g):
        noalloc()
    for sb in batches[1:]:
        logits.copy_(sb.logits.to(device))
        temp.copy_(sb.temperature.to(device))
        uni.copy_(sb.uniform.to(device))
        got.fill_(-2)
        g.replay()
        torch.cuda.synchronize()
        first = got.cpu()
        want, _ = _both(lib, logits, temp, uni)     # eager lv_sample (+ noalloc) between
        got.fill_(-2)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(first, want) and torch.equal(got.cpu(), want)
        assert torch.equal(want[:B // 2], sb.planted[:B // 2])
    del g
