"""C ABI checks that need no GPU: the library loads, exports every function
declared in include/*.h, and rejects bad arguments on the host."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(lv_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_the_four_pieces():
    names = _declared_functions()
    for fn in ("lv_pack_inputs", "lv_kv_scatter", "lv_paged_attention",
               "lv_paged_attention_workspace_size", "lv_sample", "lv_sample_workspace_size",
               "lv_last_error",
               "lv_abi_version"):
        assert fn in names


def test_library_exports_every_declared_symbol():
    from litevllm import _hip
    lib = _hip.load()
    for fn in _declared_functions():
        assert hasattr(lib, fn), fn
        assert fn in _hip.SIGNATURES, f"{fn} has no ctypes signature"
    assert lib.lv_abi_version() == _hip.ABI_VERSION


def test_host_side_argument_rejection():
    from litevllm import _hip
    lib = _hip.load()
    # null pointers / bad geometry are rejected before any launch
    rc = lib.lv_kv_scatter(None, 8, None, 8, None, None, None, 4, 2, 4, 16, 10, _hip.LV_BF16, None)
    assert rc == -1
    assert b"null pointer" in lib.lv_last_error()
    rc = lib.lv_sample(None, 4, 0, 0, None, None, None, None, 0, _hip.LV_BF16, None)
    assert rc == -1 and b"vocab_size" in lib.lv_last_error()
    rc = lib.lv_paged_attention(None, 0, None, None, 1, None, 1, None, None, 2, 3, 2, 1,
                                16, 8, 128, 16, 0.1, None, 0, None, 0, _hip.LV_BF16, None)
    assert rc == -1 and b"num_decodes" in lib.lv_last_error()
    rc = lib.lv_pack_inputs(None, 0, None, 0, None, 0, None, 0, 0, 16, 0, None, None, None,
                            None, None, None, None, None)
    assert rc == -1 and b"num_seqs" in lib.lv_last_error()
    # unsupported-but-valid request reports LV_ERR_UNSUPPORTED... only after
    # pointer checks, so a zero-size call is a clean no-op instead
    assert lib.lv_kv_scatter(None, 0, None, 0, None, None, None, 0, 1, 1, 1, 1,
                             _hip.LV_F32, None) == 0


def test_prefix_entry_host_side_checks():
    """lv_paged_attention_prefix rejects a bad plan description on the host
    (nothing is dereferenced: the pointers below are never valid memory)."""
    from litevllm import _hip
    lib = _hip.load()
    fake16, fake4 = 0x1000, 0x1004

    def call(num_decodes=8, blocks=fake16, items=fake16, max_items=4, members=fake16,
             num_members=8, pws=fake16, pws_bytes=1 << 30):
        return lib.lv_paged_attention_prefix(
            None, 0, None, None, 1, None, 1, None, None, num_decodes, num_decodes,
            num_decodes, 1, 16, 8, 128, 16, 0.1, None, 0, None, 0,
            blocks, items, max_items, members, num_members, pws, pws_bytes, _hip.LV_BF16, None)

    assert call(num_decodes=0) == -1 and b"num_decodes" in lib.lv_last_error()
    assert call(num_decodes=7001) == -1 and b"num_decodes" in lib.lv_last_error()
    assert call(blocks=None) == -1 and b"null prefix" in lib.lv_last_error()
    assert call(members=None) == -1 and b"null prefix" in lib.lv_last_error()
    assert call(items=None) == -1 and b"null prefix" in lib.lv_last_error()
    assert call(max_items=-1) == -1 and b"null prefix" in lib.lv_last_error()
    assert call(num_members=-1) == -1 and b"null prefix" in lib.lv_last_error()
    assert call(items=fake4) == -1 and b"16-byte aligned" in lib.lv_last_error()
    need = lib.lv_paged_attention_prefix_workspace_size(8, 16, 128)
    assert call(pws_bytes=need - 1) == -3 and b"prefix workspace" in lib.lv_last_error()
    assert call(pws=fake4) == -3
    # (rows, heads, 16 splits) x ((m, l) + D floats), each part 256-byte aligned
    n = 256 * 16 * 16
    assert lib.lv_paged_attention_prefix_workspace_size(256, 16, 128) == \
        -(-n * 2 * 4 // 256) * 256 + -(-n * 128 * 4 // 256) * 256
    assert lib.lv_paged_attention_prefix_workspace_size(0, 16, 128) == 0


def test_workspace_size_is_pure_host():
    from litevllm import _hip
    lib = _hip.load()
    n = lib.lv_paged_attention_workspace_size(256, 256, 256, 16, 128, 16, 128, 1, _hip.LV_BF16)
    assert n > 0 and n % 256 == 0
    # no decode rows -> no workspace; prefill rows need none
    assert lib.lv_paged_attention_workspace_size(4, 0, 400, 16, 128, 16, 64, 128, _hip.LV_BF16) == 0
    small = lib.lv_paged_attention_workspace_size(4, 4, 4, 16, 128, 16, 1, 1, _hip.LV_BF16)
    assert small > 0 and small % 256 == 0 and small <= n


def test_ops_refuse_cpu_tensors():
    import torch
    from litevllm import ops
    k = torch.zeros(2, 2, 8)
    kc = torch.zeros(4, 16, 2, 8)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        ops.kv_scatter(k, k, kc, kc.clone(), torch.zeros(2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        ops.sample(torch.zeros(2, 10), torch.zeros(2))


def test_sampler_workspace_size_and_rejection():
    from litevllm import _hip
    lib = _hip.load()
    n = lib.lv_sample_workspace_size(256, 151936)
    assert n == 256 * 297 * 8 + 256       # (maximum, sigma) per (row, segment)
    assert lib.lv_sample_workspace_size(0, 100) == 0
    assert lib.lv_sample_workspace_size(4, 0) == 0
    # too small a workspace is refused before any launch (pointers are dummies
    # that are never dereferenced on the host)
    rc = lib.lv_sample(1, 4, 1000, 1000, 1, 1, 1, 1, 8, _hip.LV_BF16, None)
    assert rc == -3 and b"workspace" in lib.lv_last_error()


def test_sample_noalloc_refuses_requests_beyond_its_scratch():
    """lv_sample_noalloc's scratch is a fixed 4 MiB: a request needing more
    is refused on the host, before any device call (none is possible here:
    this check runs without a GPU)."""
    from litevllm import _hip
    lib = _hip.load()
    p = ctypes.c_void_p(256)      # never dereferenced: the size check comes first
    need = int(lib.lv_sample_workspace_size(4096, 151936))
    assert need > 4 << 20
    rc = lib.lv_sample_noalloc(p, 4096, 151936, 151936, p, p, p, _hip.LV_BF16, None)
    assert rc == -3 and b"scratch" in lib.lv_last_error()
    assert int(lib.lv_sample_workspace_size(1765, 151936)) <= 4 << 20
    assert int(lib.lv_sample_workspace_size(1766, 151936)) > 4 << 20
    rc = lib.lv_sample_noalloc(None, 4, 100, 100, None, None, None, _hip.LV_BF16, None)
    assert rc == -1 and b"null pointer" in lib.lv_last_error()


def test_device_error_report_host_side():
    """lv_device_errors on a host without a GPU fails cleanly (LV_ERR_HIP,
    flags zeroed) instead of crashing; the Python check names every bit it
    is given."""
    from litevllm import _hip, ops
    lib = _hip.load()
    flags = ctypes.c_uint32(0xdead)
    rc = lib.lv_device_errors(ctypes.byref(flags), 1)
    if rc == 0:
        pytest.skip("a GPU is visible: the device report is covered by the -m gpu tests")
    assert rc == -2 and flags.value == 0
    assert b"lv_device_errors" in lib.lv_last_error()
    assert lib.lv_device_errors(None, 0) == -2       # NULL flags_out is allowed
    assert set(ops.DEVICE_ERROR_NAMES) == {_hip.LV_DEVERR_BLOCK_ID, _hip.LV_DEVERR_SLOT}


def test_check_device_errors_message(monkeypatch):
    from litevllm import _hip, ops
    monkeypatch.setattr(ops, "device_errors", lambda device=None, clear=True: 0)
    ops.check_device_errors()                         # nothing reported: no error
    monkeypatch.setattr(ops, "device_errors",
                        lambda device=None, clear=True: _hip.LV_DEVERR_BLOCK_ID |
                        _hip.LV_DEVERR_SLOT)
    with pytest.raises(RuntimeError, match="block-table entry.*slot_mapping entry"):
        ops.check_device_errors()
