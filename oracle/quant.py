"""numpy restatement of the W8A16 half of the hot path (test infrastructure only)."""

from __future__ import annotations

import numpy as np


def quantize(w):
    """Per-output-row symmetric int8 (quant/int8.py:8-12): scale = max|W[n, :]| / 127 clamped to
    >= 1e-8 (fp32); wq = round-half-even(W / scale) clamped to [-127, 127]."""
    w = np.asarray(w, dtype=np.float32)
    scale = np.maximum(np.abs(w).max(axis=1) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    wq = np.clip(np.round(w / scale[:, None]), -127, 127).astype(np.int8)
    return wq, scale


def dequantize(wq, scale, dtype=np.float32):
    """(wq.float() * scale[:, None]).to(dtype) (quant/int8.py:15-16)."""
    return (np.asarray(wq).astype(np.float32) * np.asarray(scale, dtype=np.float32)[:, None]).astype(dtype)


def w8a16(x, wq, scale, bias=None, acc=np.float64):
    """y = (x . wq^T) * scale[n] (+ bias[n]) with the scale applied after the contraction, as the
    Triton kernel does (ops/triton_w8a16.py:26-33); result in ``acc`` (not rounded)."""
    y = np.asarray(x).astype(acc) @ np.asarray(wq).astype(acc).T
    y = y * np.asarray(scale).astype(acc)[None, :]
    if bias is not None:
        y = y + np.asarray(bias).astype(acc)[None, :]
    return y


def linear_twin(x, wq, scale, bias=None):
    """The twin's order (ops/reference.py:45-47): dequantise to the activation dtype (fp16), then
    the product, accumulated here in fp32 and rounded to fp16."""
    w16 = dequantize(wq, scale, np.float16)
    y = np.asarray(x).astype(np.float32) @ w16.astype(np.float32).T
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32)[None, :]
    return y.astype(np.float16)
