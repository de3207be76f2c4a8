"""The fused gated-MLP activation (ts_w8a16_glu) on the GPU: silu(gate) * up straight out of the
gate_up W8A16 product (model/qwen2.py:35-36 with ops/triton_silu_mul.py:21-28).

It must equal, bit for bit, the unfused pair it replaces -- the W8A16 product of the [M, 2I]
shape with the same variant and splits, then silu_mul -- over every path the plan can take
(weight streaming, skinny, 128 x 64 and 128 x 128 tiles, split-K), ragged shapes and bias; and
that pair is pinned to the float64 oracle of the product (oracle/quant.py) composed with
silu * up.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant as OQ
from turingserve_amd import hip_ops as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _problem(M, inter, Kd, seed, bias=False, fp16_scale=False):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(2 * inter, Kd, generator=g) * 0.05
    wq, sc = OQ.quantize(w.numpy())
    x = torch.randn(M, Kd, generator=g).half()
    b = (torch.randn(2 * inter, generator=g) * 0.1).half() if bias else None
    scale = torch.from_numpy(sc)
    if fp16_scale:
        scale = scale.half()
    return (x.to(DEV), torch.from_numpy(wq).to(DEV), scale.to(DEV),
            None if b is None else b.to(DEV), wq, sc, b)


def _unfused(x, wq, scale, b, cfg):
    return K.silu_mul(K.w8a16_linear(x, wq, scale, b, cfg))


@pytest.mark.parametrize("M,inter,Kd", [
    (1, 8960, 1536), (16, 8960, 1536), (64, 8960, 1536), (560, 8960, 1536),   # 1.5B gate_up
    (2048, 8960, 1536), (300, 4864, 896),                                      # 0.5B gate_up
    (7, 104, 200), (130, 104, 200), (33, 40, 64), (5, 8, 8)])                  # I % 64, K % 64
def test_glu_equals_gemm_then_silu_mul(M, inter, Kd):
    x, wq, scale, _, _, _, _ = _problem(M, inter, Kd, seed=M + inter + Kd)
    fused = K.w8a16_glu(x, wq, scale)
    assert fused.shape == (M, inter) and fused.dtype == torch.float16
    assert torch.equal(fused, _unfused(x, wq, scale, None, None))


def _ulp(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in fp16 units in the last place (same-sign values; 0 for equal bits)."""
    ia, ib = a.view(torch.int16).int(), b.view(torch.int16).int()
    key = lambda i: torch.where(i < 0, -(i & 0x7FFF), i)
    return (key(ia) - key(ib)).abs()


@pytest.mark.parametrize("M,inter", [(7, 100), (130, 36), (40, 4)])
def test_glu_intermediate_not_a_multiple_of_8(M, inter):
    """Output rows whose length is not a multiple of 8 (or 4: the last four-column store is
    split), which the separate silu_mul kernel does not take: the fused result must be the
    fp16 roundings of silu_mul applied to the product -- silu(g) in float64 rounded to fp16,
    times u rounded to fp16 -- up to the fp32 exponential: at most 1 ulp, almost all exact."""
    x, wq, scale, _, _, _, _ = _problem(M, inter, 200, seed=M * inter)
    fused = K.w8a16_glu(x, wq, scale)
    gu = K.w8a16_linear(x, wq, scale, None)
    gf, up = gu[:, :inter].double(), gu[:, inter:].double()
    want = ((gf / (1 + torch.exp(-gf))).half().double() * up).half()
    d = _ulp(fused, want)
    assert torch.isfinite(fused).all()
    assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99


@pytest.mark.parametrize("variant,splits", [(1, 0), (1, 1), (1, 3), (2, 0), (2, 1), (2, 4),
                                            (3, 0), (3, 2), (4, 0), (4, 2), (5, 0), (6, 0),
                                            (6, 2), (7, 0)])
@pytest.mark.parametrize("M", [3, 9, 32, 200])
def test_glu_every_variant_and_split(variant, splits, M):
    if variant == 7 and M > 4:
        pytest.skip("the VALU path is built for M <= 4")
    if variant == 1 and M > 32:
        pytest.skip("weight streaming is built for M <= 32")
    if variant == 5 and M > 64:
        pytest.skip("the skinny kernel is built for M <= 64")
    x, wq, scale, b, _, _, _ = _problem(M, 1000, 1024, seed=variant * 10 + splits + M, bias=True,
                                        fp16_scale=True)
    cfg = (variant, splits)
    # (variant 4 runs as 128 x 64 tiles in GLU mode and as 128 x 32 tiles unfused: every output
    # element is summed over K in the same order either way, so the results are still equal)
    assert torch.equal(K.w8a16_glu(x, wq, scale, b, cfg), _unfused(x, wq, scale, b, cfg))


def test_glu_matches_float64_oracle():
    x, wq, scale, b, wq_np, sc_np, b_np = _problem(70, 300, 512, seed=3, bias=True)
    out = K.w8a16_glu(x, wq, scale, b).double().cpu().numpy()
    gu = OQ.w8a16(x.cpu().numpy(), wq_np, sc_np, b_np.numpy(), np.float64)
    gate, up = gu[:, :300], gu[:, 300:]
    ref = gate / (1.0 + np.exp(-gate)) * up
    # three fp16 roundings (gate / up, silu, product) on values of order 1
    assert np.max(np.abs(out - ref)) < 2e-2
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 2e-3


def test_glu_empty_and_model_routing():
    from turingserve_amd import get_ops
    from turingserve_amd.qwen2 import TINY_G2, random_weights

    x, wq, scale, _, _, _, _ = _problem(3, 64, 64, seed=1)
    assert K.w8a16_glu(x[:0], wq, scale).shape == (0, 64)
    ops = get_ops("hip")
    h = torch.randn(11, TINY_G2.hidden_size, device=DEV).half()
    for quantization in ("int8", "none"):                 # fused call / the two calls
        lw = random_weights(TINY_G2, DEV, seed=4, quantization=quantization).layers[0].gate_up_proj
        assert lw.quantized == (quantization == "int8")
        got = ops.gate_up_silu(h, lw)
        assert torch.equal(got, ops.silu_mul(ops.linear(h, lw)))
