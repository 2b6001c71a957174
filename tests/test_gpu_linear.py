"""lv_linear (decode-sized linear layers on MFMA) against float32 products of
the same bf16/fp16 operands.

A library GEMM rounds the fp32 sum once to the dtype, so both lv_linear and
torch's GEMM sit within one rounding of the fp32 product (relative 2^-8 for
bf16); the bound used is 1.5 units in the last place of the output plus the
fp32 summation-order slack."""

from __future__ import annotations

import os

import pytest
import torch

from litevllm import ops

pytestmark = pytest.mark.gpu

SHAPES = [  # (N, K): qkv, o, gate_up, down of the Qwen3-0.6B shape, a small lm_head
    (4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (32000, 1024)]


def _ulp(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Spacing of `dtype` values at |t| (t in float32)."""
    mant = 8 if dtype == torch.bfloat16 else 11
    e = torch.floor(torch.log2(t.float().abs().clamp_min(1e-30)))
    return torch.pow(2.0, e - (mant - 1))


def _check(got: torch.Tensor, ref32: torch.Tensor, k: int, scale: torch.Tensor) -> None:
    err = (got.float() - ref32).abs()
    # output rounding (<= 1 ulp of the value; 1.5 allows the value near a
    # binade edge) + fp32 accumulation slack ~ k * 2^-24 * sum |x w|
    bound = 1.5 * _ulp(ref32, got.dtype) + k * 2.0 ** -22 * scale + 1e-6
    bad = err > bound
    assert not bad.any(), (f"{int(bad.sum())} of {err.numel()} beyond bound; "
                           f"max err {err.max():.3e}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 7, 64, 200, 256])
@pytest.mark.parametrize("nk", SHAPES)
def test_linear_matches_fp32_product(dtype, m, nk):
    n, k = nk
    g = torch.Generator(device="cuda").manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, device="cuda", generator=g).to(dtype)
    w = (torch.randn(n, k, device="cuda", generator=g) * k ** -0.5).to(dtype)
    assert ops.linear_supported(m, n, k, dtype)
    y = ops.linear(x, w)
    ref = x.float() @ w.float().T
    scale = x.float().abs() @ w.float().abs().T
    _check(y, ref, k, scale)
    torch.cuda.synchronize()


@pytest.mark.parametrize("cfg", ["0", "1", "2", "3"])
def test_every_tile_shape_gives_the_same_sums(cfg, monkeypatch):
    """Each forced tile configuration is within the bound of the fp32
    product; ragged m exercises the clamped rows."""
    n, k, m = 1024, 2048, 77
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, device="cuda", generator=g) * k ** -0.5).to(torch.bfloat16)
    monkeypatch.setenv("LV_LINEAR_CFG", cfg)
    y = ops.linear(x, w)
    monkeypatch.delenv("LV_LINEAR_CFG")
    ref = x.float() @ w.float().T
    _check(y, ref, k, x.float().abs() @ w.float().abs().T)


def test_strided_rows_and_out_buffer():
    n, k, m = 4096, 1024, 33
    x_big = torch.randn(m, k + 64, device="cuda").to(torch.bfloat16)
    x = x_big[:, 32:32 + k]
    w = (torch.randn(n, k, device="cuda") * k ** -0.5).to(torch.bfloat16)
    out_big = torch.full((m, n + 32), 7.0, device="cuda", dtype=torch.bfloat16)
    out = out_big[:, :n]
    ops.linear(x, w, out=out)
    ref = x.float() @ w.float().T
    _check(out, ref, k, x.float().abs() @ w.float().abs().T)
    assert torch.all(out_big[:, n:] == 7.0)


def test_unsupported_shapes_raise_and_report():
    assert not ops.linear_supported(8, 100, 1024, torch.bfloat16)   # n % 32
    assert not ops.linear_supported(8, 100, 1024, torch.bfloat16, "silu_mul")
    assert not ops.linear_supported(8, 1024, 1000, torch.bfloat16)  # k % 128
    assert not ops.linear_supported(8, 1024, 1024, torch.float32)
    x = torch.randn(8, 1000, device="cuda").to(torch.bfloat16)
    w = torch.randn(1024, 1000, device="cuda").to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="no kernel"):
        ops.linear(x, w)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 64, 200, 256])
@pytest.mark.parametrize("cfg", ["0", "1"])
def test_silu_mul_epilogue_equals_plain_then_silu_mul(dtype, m, cfg, monkeypatch):
    """The fused gate|up + SiLU form gives exactly lv_silu_mul of the plain
    product (same k order of the sums), and is within rounding of the fp32
    composition silu(x g^T) * (x u^T)."""
    inter, k = 3072, 1024
    g = torch.Generator(device="cuda").manual_seed(m + 11)
    x = torch.randn(m, k, device="cuda", generator=g).to(dtype)
    w = (torch.randn(2 * inter, k, device="cuda", generator=g) * k ** -0.5).to(dtype)
    assert ops.linear_supported(m, inter, k, dtype, "silu_mul")
    monkeypatch.setenv("LV_LINEAR_SILU_CFG", cfg)
    fused = ops.linear(x, w, activation="silu_mul")
    monkeypatch.delenv("LV_LINEAR_SILU_CFG")
    plain = ops.linear(x, w)
    assert torch.equal(fused, ops.silu_mul(plain))
    ref = x.float() @ w.float().T
    gate, up = ref[:, :inter], ref[:, inter:]
    want = torch.nn.functional.silu(gate) * up
    err = (fused.float() - want).abs()
    tol = (4 * _ulp(want, dtype) + 4 * _ulp(up, dtype) * (gate.abs() + 1)
           + 2 * _ulp(gate, dtype) * up.abs() + 1e-5)
    assert (err <= tol).all(), err.max()
