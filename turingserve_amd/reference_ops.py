"""The ``reference`` op namespace: pure-PyTorch twins of every op (CPU or GPU).

These restate ops/reference.py:13-111 with the same numerics (fp32 math where the twins use it,
the HF cast order for the norms), so ``get_ops("reference")`` behaves like the reference's
``--kernels reference`` switch. They are slow and simple; the ``hip`` namespace is checked
against them.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from turingserve_amd.quant import LinearWeight, dequantize


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMS in fp32, cast back to x.dtype, then times the weight (ops/reference.py:13-16)."""
    x32 = x.float()
    y = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    return w * y.to(x.dtype)


def rmsnorm_residual(x: torch.Tensor, residual: torch.Tensor | None, w: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """residual <- x + residual (in x.dtype), out = rmsnorm(residual) (ops/reference.py:19-23)."""
    new_res = x if residual is None else x + residual
    return rmsnorm(new_res, w, eps), new_res


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for gu = [gate | up] (ops/reference.py:26-28)."""
    i = gu.shape[-1] // 2
    return F.silu(gu[..., :i]) * gu[..., i:]


def rope_(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
          H: int, KVH: int, D: int) -> None:
    """In-place rotate-half RoPE on the q and k heads of qkv [T, (H + 2 KVH) D]; the fp32 tables
    are cast to the activation dtype first (ops/reference.py:31-42)."""
    T = qkv.shape[0]
    c = cos[positions].to(qkv.dtype)[:, None, :]
    s = sin[positions].to(qkv.dtype)[:, None, :]
    qk = qkv[:, : (H + KVH) * D].view(T, H + KVH, D)
    half = D // 2
    x1, x2 = qk[..., :half], qk[..., half:]
    o1 = x1 * c - x2 * s
    o2 = x2 * c + x1 * s
    qk[..., :half] = o1
    qk[..., half:] = o2


def linear(x: torch.Tensor, lw: LinearWeight) -> torch.Tensor:
    """Dequantise to x.dtype (if int8), then F.linear (ops/reference.py:45-47)."""
    w = dequantize(lw.w, lw.scale, x.dtype) if lw.quantized else lw.w
    return F.linear(x, w, lw.b)


def kv_write(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             slot_mapping: torch.Tensor) -> None:
    """cache[slot // 16, :, slot % 16, :] = row for slot >= 0 (ops/reference.py:50-57)."""
    keep = slot_mapping >= 0
    slots = slot_mapping[keep]
    blk, off = slots // 16, slots % 16
    k_cache[blk, :, off, :] = k[keep]
    v_cache[blk, :, off, :] = v[keep]


def attention_with_mask(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        scale: float) -> torch.Tensor:
    """q [Tq, H, D], k/v [Tk, KVH, D] -> [Tq, H*D]; fp32 math with an explicit bottom-right
    causal mask j <= (Tk - Tq) + i (ops/reference.py:60-77)."""
    Tq, H, D = q.shape
    Tk, KVH, _ = k.shape
    G = H // KVH
    qf = q.float().permute(1, 0, 2)
    kf = k.float().repeat_interleave(G, dim=1).permute(1, 0, 2)
    vf = v.float().repeat_interleave(G, dim=1).permute(1, 0, 2)
    scores = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale
    i = torch.arange(Tq, device=q.device)[:, None]
    j = torch.arange(Tk, device=q.device)[None, :]
    scores = scores.masked_fill(~(j <= (Tk - Tq) + i), float("-inf"))
    p = torch.softmax(scores, dim=-1)
    out = torch.matmul(p, vf).permute(1, 0, 2)
    return out.reshape(Tq, H * D).to(q.dtype)


def dense_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           scale: float) -> torch.Tensor:
    """Causal attention with q_len == kv_len (ops/reference.py:80-91)."""
    T, H, D = q.shape
    G = H // k.shape[1]
    kk = k.repeat_interleave(G, dim=1)
    vv = v.repeat_interleave(G, dim=1)
    out = F.scaled_dot_product_attention(
        q.permute(1, 0, 2)[None], kk.permute(1, 0, 2)[None], vv.permute(1, 0, 2)[None],
        is_causal=True, scale=scale)
    return out[0].permute(1, 0, 2).reshape(T, H * D)


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, meta,
                    scale: float) -> torch.Tensor:
    """Per-sequence gather of the paged cache, then attention_with_mask; rows of sequences with
    seq_len 0 stay 0 (ops/reference.py:94-111)."""
    T, H, D = q.shape
    KVH = k_cache.shape[1]
    out = torch.zeros(T, H * D, dtype=q.dtype, device=q.device)
    qsl = meta.query_start_loc.tolist()
    for b, seq_len in enumerate(meta.seq_lens.tolist()):
        qs, qe = qsl[b], qsl[b + 1]
        if seq_len == 0 or qe == qs:
            continue
        nb = -(-seq_len // 16)
        blocks = meta.block_tables[b, :nb].long()
        kk = k_cache[blocks].permute(0, 2, 1, 3).reshape(nb * 16, KVH, D)[:seq_len]
        vv = v_cache[blocks].permute(0, 2, 1, 3).reshape(nb * 16, KVH, D)[:seq_len]
        out[qs:qe] = attention_with_mask(q[qs:qe], kk, vv, scale)
    return out
