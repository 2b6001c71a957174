"""Fused layer kernels (lv_add_rms_norm, lv_qk_norm_rope_cache, lv_silu_mul)
against the CPU oracle that replays the reference's torch ops.

Tolerance: results may differ from the reference by the rounding of one
intermediate (the fp32 sum of squares is reduced in another order and rsqrt
is another routine), i.e. by 1-2 units in the last place of the dtype, on
few elements: |got - want| <= 2 ulp(|want|) everywhere and exact on >= 95%
(bf16/fp16) of the elements; fp32 within 1e-5 relative.  The V half of the
cache write is a copy and must be bit-exact."""

from __future__ import annotations

import pytest
import torch

from litevllm import ops
from oracle import layers as L

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _close(got: torch.Tensor, want: torch.Tensor, dtype: torch.dtype, exact_frac: float = 0.95,
           scale: torch.Tensor | None = None):
    """`scale` (default |want|) sets the magnitude whose ulp bounds the error."""
    got, want = got.float().cpu(), want.float().cpu()
    assert got.shape == want.shape
    mag = want.abs() if scale is None else scale.float().cpu()
    if dtype == torch.float32:
        assert ((got - want).abs() <= 1e-5 * mag + 1e-6).all(), (got - want).abs().max()
        return
    mant = 7 if dtype == torch.bfloat16 else 10
    ulp = torch.exp2(torch.floor(torch.log2(mag.clamp_min(1e-30))) - mant)
    assert ((got - want).abs() <= 2 * ulp + 1e-30).all(), (got - want).abs().max()
    assert (got == want).float().mean() >= exact_frac


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,hidden", [(1, 256), (37, 1024), (256, 1024), (5, 4096), (3, 24)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_add_rms_norm_matches_oracle(device, dtype, T, hidden, with_residual):
    if hidden * torch.tensor([], dtype=dtype).element_size() % 16:
        pytest.skip("hidden must be a multiple of 16 bytes")
    _say(f"add_rms_norm {dtype} T={T} hidden={hidden} residual={with_residual}")
    g = torch.Generator().manual_seed(T * 7 + hidden)
    x = (torch.randn(T, hidden, generator=g) * 3).to(dtype)
    r = torch.randn(T, hidden, generator=g).to(dtype) if with_residual else None
    w = (torch.rand(hidden, generator=g) + 0.5).to(dtype)
    want, want_res = L.add_rms_norm(x, r, w, 1e-6)
    rd = r.to(device) if r is not None else None
    got = ops.add_rms_norm(x.to(device), w.to(device), 1e-6, residual=rd)
    _close(got, want, dtype)
    if with_residual:
        assert torch.equal(rd.cpu(), want_res)   # the bf16 sum is exact-rounded: bit-exact


def test_add_rms_norm_strided_rows_and_errors(device):
    _say("add_rms_norm strided / errors")
    x = torch.randn(8, 2048, device=device, dtype=torch.bfloat16)[:, :1024]
    w = torch.ones(1024, device=device, dtype=torch.bfloat16)
    want, _ = L.add_rms_norm(x.cpu(), None, w.cpu(), 1e-5)
    _close(ops.add_rms_norm(x, w, 1e-5), want, torch.bfloat16)
    with pytest.raises(RuntimeError):
        ops.add_rms_norm(x, torch.ones(1000, device=device, dtype=torch.bfloat16), 1e-5)
    assert ops.add_rms_norm(x[:0], w, 1e-5).shape == (0, 1024)


def _rope_tables(D, P, dtype, theta=1e6):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D)
    f = torch.outer(torch.arange(P, dtype=torch.float32), inv)
    return f.cos().to(dtype), f.sin().to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("H,Hkv,D", [(16, 8, 128), (4, 2, 64), (8, 1, 256), (32, 8, 64)])
@pytest.mark.parametrize("qk_norm", [True, False])
def test_qk_norm_rope_cache_matches_oracle(device, dtype, H, Hkv, D, qk_norm):
    _say(f"qk_norm_rope_cache {dtype} H={H} Hkv={Hkv} D={D} norm={qk_norm}")
    g = torch.Generator().manual_seed(H * 1000 + D)
    T, bs, nb, P = 45, 16, 12, 4096
    qkv = torch.randn(T, (H + 2 * Hkv) * D, generator=g).to(dtype)
    cos, sin = _rope_tables(D, P, dtype)
    pos = torch.randint(0, P, (T,), generator=g)
    slots = torch.randperm(nb * bs, generator=g)[:T]
    slots[3] = -1                                   # padding token
    qw = (torch.rand(D, generator=g) + 0.5).to(dtype) if qk_norm else None
    kw = (torch.rand(D, generator=g) + 0.5).to(dtype) if qk_norm else None
    kc = torch.full((nb, bs, Hkv, D), 3.0, dtype=dtype)
    vc = torch.full((nb, bs, Hkv, D), 3.0, dtype=dtype)
    kc_d, vc_d = kc.to(device), vc.to(device)
    want_q = L.qk_norm_rope_cache(qkv, H, Hkv, D, cos, sin, pos, slots, kc, vc, qw, kw, 1e-6)
    dv = lambda t: None if t is None else t.to(device)
    got_q = ops.qk_norm_rope_cache(dv(qkv), H, Hkv, D, dv(cos), dv(sin), dv(pos), dv(slots), kc_d,
                                   vc_d, q_norm_weight=dv(qw), k_norm_weight=dv(kw), eps=1e-6)
    # a rotated element is a difference/sum of two products: a 1-ulp change
    # of a normalised input can move it by an ulp of the pair's magnitude
    # (the rotation keeps that magnitude), not of the (possibly cancelled)
    # element itself
    def pair_mag(x):
        x = x.float()
        a, b = x.chunk(2, dim=-1)
        m = (a * a + b * b).sqrt()
        return torch.cat([m, m], dim=-1)
    _close(got_q, want_q, dtype, scale=pair_mag(want_q))
    _close(kc_d, kc, dtype, exact_frac=0.95, scale=pair_mag(kc))
    assert torch.equal(vc_d.cpu(), vc)


def test_qk_norm_rope_cache_position_zero_is_copy(device):
    _say("qk_norm_rope_cache position 0")
    H, Hkv, D = 2, 1, 128
    qkv = torch.randn(3, (H + 2 * Hkv) * D, device=device, dtype=torch.bfloat16)
    cos, sin = _rope_tables(D, 8, torch.bfloat16)
    kc = torch.zeros(1, 16, Hkv, D, device=device, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    pos = torch.zeros(3, dtype=torch.int64, device=device)
    q = ops.qk_norm_rope_cache(qkv, H, Hkv, D, cos.to(device), sin.to(device), pos,
                               torch.arange(3, device=device), kc, vc)
    assert torch.equal(q.reshape(3, -1), qkv[:, :H * D])
    assert torch.equal(kc[0, :3].reshape(3, -1), qkv[:, H * D:(H + Hkv) * D])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("T,inter", [(1, 688), (256, 3072), (77, 512), (8192, 3072)])
def test_silu_mul_matches_oracle(device, dtype, T, inter):
    if inter * torch.tensor([], dtype=dtype).element_size() % 16:
        pytest.skip("intermediate must be a multiple of 16 bytes")
    _say(f"silu_mul {dtype} T={T} inter={inter}")
    g = torch.Generator().manual_seed(T + inter)
    gu = (torch.randn(T, 2 * inter, generator=g) * 4).to(dtype)
    want = L.silu_mul(gu)
    got = ops.silu_mul(gu.to(device))
    _close(got, want, dtype, exact_frac=0.98)
