"""Fused small ops on the GPU (ts_rmsnorm, ts_rope, ts_silu_mul) against the torch twins of
ops/reference.py:13-42 and against float64 restatements of the reference kernels' rounding
(ops/triton_rmsnorm.py:10-27, ops/triton_rope.py:10-24, ops/triton_silu_mul.py:10-18).

RoPE repeats the twin's fp16 arithmetic and must match it bit for bit. RMSNorm and SiLU.up reduce
or exponentiate in fp32 in another order than torch, so their bar is a distance in fp16 units in
the last place (ulp) from the float64 restatements and from the twins: at most 2 ulp, bit-exact
on at least 97-99% of elements."""

from __future__ import annotations

import pytest
import torch

from turingserve_amd import get_ops
from turingserve_amd import hip_ops as H
from turingserve_amd import reference_ops as R
from turingserve_amd.qwen2 import rope_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance between fp16 values counted in representable steps (sign-magnitude order)."""
    def key(x):
        i = x.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (key(a) - key(b)).abs()


def assert_ulp(got: torch.Tensor, want: torch.Tensor, max_ulp: int, min_exact: float, what: str):
    assert got.shape == want.shape and got.dtype == want.dtype == torch.float16, what
    assert torch.isfinite(got).all(), what
    d = ulp_distance(got, want)
    exact = float((d == 0).float().mean())
    assert int(d.max()) <= max_ulp and exact >= min_exact, \
        f"{what}: max {int(d.max())} ulp, {exact:.4f} bit-exact"


@pytest.mark.parametrize("T,N", [(1, 64), (7, 224), (560, 1536), (33, 896), (5, 8192)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_matches_twin(T, N, with_residual):
    g = torch.Generator(device=DEV).manual_seed(T * 131 + N)
    x = (torch.randn(T, N, generator=g, device=DEV) * 3).half()
    res = (torch.randn(T, N, generator=g, device=DEV) * 3).half() if with_residual else None
    w = (1 + 0.1 * torch.randn(N, generator=g, device=DEV)).half()
    out, new_res = H.rmsnorm_residual(x, res, w, 1e-6)
    r_out, r_res = R.rmsnorm_residual(x, res, w, 1e-6)
    assert torch.equal(new_res, r_res), "residual sum must be the fp16 add, bit-exact"
    if res is None:
        assert new_res.data_ptr() == x.data_ptr()
    # float64 restatement of the kernel's rounding: RMS of the rounded sum, cast, times w
    r64 = new_res.double()
    y = (r64 * torch.rsqrt(r64.pow(2).mean(-1, keepdim=True) + 1e-6)).half()
    want = (w.double() * y.double()).half()
    # two roundings (the normalised row, then the weight product) after an fp32 rsqrt: a value
    # on a rounding boundary can land 2 ulp away from the float64 result
    assert_ulp(out, want, 2, 0.99, f"rmsnorm vs float64 T={T} N={N}")
    assert_ulp(out, r_out, 2, 0.97, f"rmsnorm vs twin T={T} N={N}")


def test_rmsnorm_strided_rows_and_plain_entry():
    g = torch.Generator(device=DEV).manual_seed(3)
    big = (torch.randn(16, 2048, generator=g, device=DEV)).half()
    x = big[:, :1536]                                    # row stride 2048, unit column stride
    w = torch.ones(1536, dtype=torch.float16, device=DEV)
    assert_ulp(H.rmsnorm(x, w, 1e-6), R.rmsnorm(x, w, 1e-6), 2, 0.97, "strided rmsnorm")


@pytest.mark.parametrize("T,Hq,KVH,D", [(560, 12, 2, 128), (9, 4, 2, 16), (5, 14, 2, 64),
                                        (3, 2, 1, 8)])
def test_rope_matches_twin_in_place(T, Hq, KVH, D):
    g = torch.Generator(device=DEV).manual_seed(T + D)
    cos, sin = rope_tables(D, 1e6, 4096, DEV)
    qkv = (torch.randn(T, (Hq + 2 * KVH) * D, generator=g, device=DEV)).half()
    pos = torch.randint(0, 4096, (T,), generator=g, device=DEV)
    ours, twin = qkv.clone(), qkv.clone()
    H.rope_(ours, pos, cos, sin, Hq, KVH, D)
    R.rope_(twin, pos, cos, sin, Hq, KVH, D)
    nqk = (Hq + KVH) * D
    assert torch.equal(ours[:, nqk:], qkv[:, nqk:]), "v heads must be untouched"
    # float64 restatement of the twin's fp16 arithmetic: tables, products and sums each rounded
    c = cos[pos].half().double()[:, None, :]
    s = sin[pos].half().double()[:, None, :]
    qk = qkv[:, :nqk].view(T, Hq + KVH, D).double()
    x1, x2 = qk[..., : D // 2], qk[..., D // 2:]
    # (fp16 products are exact in float64; each sum is formed in fp32, then rounded to fp16,
    # which is what the twin's fp16 add does on the GPU)
    r = lambda v: v.half().double()
    f = lambda v: v.float().half()
    want = torch.cat([f(r(x1 * c) - r(x2 * s)), f(r(x2 * c) + r(x1 * s))], -1).view(T, nqk)
    assert torch.equal(ours[:, :nqk], want), f"rope vs float64 restatement D={D}"
    assert torch.equal(ours, twin), f"rope vs twin D={D}"


def test_rope_position_zero_is_identity_and_clamps():
    cos, sin = rope_tables(128, 1e6, 64, DEV)
    qkv = torch.randn(4, 16 * 128, device=DEV).half()
    ours = qkv.clone()
    H.rope_(ours, torch.zeros(4, dtype=torch.int64, device=DEV), cos, sin, 12, 2, 128)
    assert torch.equal(ours, qkv)                        # cos 0 = 1, sin 0 = 0
    # positions past the table are clamped to its last row instead of reading past it
    a, b = qkv.clone(), qkv.clone()
    H.rope_(a, torch.full((4,), 63, dtype=torch.int64, device=DEV), cos, sin, 12, 2, 128)
    H.rope_(b, torch.full((4,), 10_000, dtype=torch.int64, device=DEV), cos, sin, 12, 2, 128)
    assert torch.equal(a, b)


@pytest.mark.parametrize("T,I", [(1, 8960), (560, 8960), (7, 128), (3, 448)])
def test_silu_mul_matches_twin(T, I):
    g = torch.Generator(device=DEV).manual_seed(T * 7 + I)
    gu = (torch.randn(T, 2 * I, generator=g, device=DEV) * 4).half()
    out = H.silu_mul(gu)
    gf = gu[:, :I].double()
    want = ((gf / (1 + torch.exp(-gf))).half().double() * gu[:, I:].double()).half()
    # two roundings (silu, then the product) after an fp32 exp: 2 ulp at a rounding boundary
    assert_ulp(out, want, 2, 0.99, f"silu_mul vs float64 I={I}")
    assert_ulp(out, R.silu_mul(gu), 2, 0.99, f"silu_mul vs twin I={I}")


def test_hip_namespace_routes_small_ops_to_kernels():
    ns = get_ops("hip")
    assert ns.rmsnorm is H.rmsnorm and ns.rmsnorm_residual is H.rmsnorm_residual
    assert ns.rope_ is H.rope_ and ns.silu_mul is H.silu_mul
