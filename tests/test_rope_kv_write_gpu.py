"""RoPE fused with the cache write (ts_rope_kv_write) on the GPU: one pass per token row must
leave qkv and both caches exactly as rope_ followed by kv_write do (the per-layer sequence of
model/qwen2.py:26-28 and :89), padding slots (-1) and out-of-range slots included; and kv_write's
part is pinned to the oracle's cache write (oracle/paged.py) of the rotated rows."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged as OP
from turingserve_amd import hip_ops as K
from turingserve_amd.qwen2 import rope_tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("H,KVH,D", [(12, 2, 128), (14, 2, 64), (4, 2, 16), (8, 8, 64)])
@pytest.mark.parametrize("T", [1, 64, 560])
def test_rope_kv_write_equals_rope_then_kv_write(H, KVH, D, T):
    g = torch.Generator().manual_seed(T * 7 + H + D)
    NB = 64 + T // 16
    qkv = (torch.randn(T, (H + 2 * KVH) * D, generator=g) * 2).half().to(DEV)
    pos = torch.randint(0, 4000, (T,), generator=g).to(DEV)
    slots = torch.randperm(NB * 16, generator=g)[:T].long()
    slots[::7] = -1                                   # padding rows
    if T > 1:
        slots[1] = NB * 16 + 5                        # out of range: skipped like -1
    slots = slots.to(DEV)
    cos, sin = rope_tables(D, 1e6, 4096, DEV)
    kc = torch.randn(NB, KVH, 16, D, generator=g).half().to(DEV)
    vc = torch.randn(NB, KVH, 16, D, generator=g).half().to(DEV)
    qkv1, kc1, vc1 = qkv.clone(), kc.clone(), vc.clone()
    assert K.rope_kv_write_(qkv1, pos, cos, sin, H, KVH, D, kc1, vc1, slots)
    qkv2, kc2, vc2 = qkv.clone(), kc.clone(), vc.clone()
    K.rope_(qkv2, pos, cos, sin, H, KVH, D)
    k2 = qkv2[:, H * D:(H + KVH) * D].view(T, KVH, D)
    v2 = qkv2[:, (H + KVH) * D:].view(T, KVH, D)
    K.kv_write(k2, v2, kc2, vc2, slots)
    assert torch.equal(qkv1, qkv2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    kn, vn = kc.cpu().numpy().copy(), vc.cpu().numpy().copy()
    sl = slots.cpu().numpy().copy()
    sl[sl >= NB * 16] = -1                            # the library skips these like -1
    OP.kv_write(k2.cpu().numpy(), v2.cpu().numpy(), kn, vn, sl)
    assert np.array_equal(kc1.cpu().numpy(), kn) and np.array_equal(vc1.cpu().numpy(), vn)


def test_rope_kv_write_declines_unaligned_rows():
    H, KVH, D = 4, 2, 16
    cos, sin = rope_tables(D, 1e6, 64, DEV)
    base = torch.zeros(3, (H + 2 * KVH) * D + 4, dtype=torch.float16, device=DEV)
    qkv = base[:, 4:]                                 # rows start 8 bytes past 16-byte alignment
    kc = torch.zeros(4, KVH, 16, D, dtype=torch.float16, device=DEV)
    before = qkv.clone()
    assert not K.rope_kv_write_(qkv, torch.zeros(3, dtype=torch.int64, device=DEV), cos,
                                sin, H, KVH, D, kc, kc.clone(),
                                torch.zeros(3, dtype=torch.int64, device=DEV))
    assert torch.equal(qkv, before)                   # declined: nothing was done
