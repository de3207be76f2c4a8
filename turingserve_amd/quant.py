"""The W8A16 weight format: per-output-row symmetric int8 with an fp32 scale.

Restates quant/int8.py:8-16 and the LinearWeight container of model/layers.py:21-31. The GEMM
also accepts fp16 scales (the W8A16 benchmark configuration draws them in fp16; widening fp16
to fp32 is exact).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class LinearWeight:
    """``w`` is [N, K] fp16/fp32, or int8 with a per-row ``scale`` [N] (W8A16); ``b`` [N] or None."""

    w: torch.Tensor
    b: torch.Tensor | None = None
    scale: torch.Tensor | None = None

    @property
    def quantized(self) -> bool:
        return self.scale is not None


def quantize(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """W [N, K] -> (int8 [N, K], fp32 scale [N]); scale = max|W[n, :]| / 127 clamped to 1e-8."""
    scale = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8).float()
    wq = torch.round(w / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return wq, scale


def dequantize(wq: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return (wq.to(torch.float32) * scale.float()[:, None]).to(dtype)
