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


# ------------------------------------------------------------------------------------------
# The qkv product with RoPE and the cache write in its epilogue (ts_w8a16_qkv_rope_kv_write)
# ------------------------------------------------------------------------------------------
def _qkv_problem(M, H, KVH, D, Kd, seed):
    from turingserve_amd.quant import LinearWeight, quantize

    g = torch.Generator().manual_seed(seed)
    Nn = (H + 2 * KVH) * D
    w = torch.randn(Nn, Kd, generator=g) * 0.05
    wq, sc = quantize(w)
    bias = (torch.randn(Nn, generator=g) * 0.1).half()
    lw = LinearWeight(wq.to(DEV), bias.to(DEV), sc.to(DEV))
    x = torch.randn(M, Kd, generator=g).half().to(DEV)
    NB = 64 + M // 8
    pos = torch.randint(-3, 4100, (M,), generator=g)          # some outside the table
    slots = torch.randperm(NB * 16, generator=g)[:M].long()
    slots[::5] = -1                                           # padding rows
    if M > 2:
        slots[2] = NB * 16 + 3                                # past the cache: not written
    kc = torch.randn(NB, KVH, 16, D, generator=g).half().to(DEV)
    vc = torch.randn(NB, KVH, 16, D, generator=g).half().to(DEV)
    return x, lw, pos.to(DEV), slots.to(DEV), kc, vc


@pytest.mark.parametrize("M,H,KVH,D,Kd,cfg", [
    (560, 12, 2, 128, 1536, None),     # config 5's qkv: 128 x 64 tiles, fused epilogue
    (2048, 12, 2, 128, 1536, None),    # a prefill chunk: 128 x 128 tiles
    (300, 12, 2, 128, 1536, (6, 0)),   # 128 x 192 tiles
    (100, 12, 2, 128, 1536, (4, 0)),   # 128 x 32 tiles
    (77, 4, 1, 128, 512, (2, 2)),      # split K: the product then rope_kv_write
    (5, 12, 2, 128, 1536, None),       # small M: the streaming / skinny kernels, two launches
    (560, 14, 2, 64, 896, None),       # head_dim 64: two launches
    (200, 12, 2, 128, 1000, None),     # K % 64 != 0: the register-path kernel, two launches
])
def test_qkv_rope_kv_write_equals_the_separate_calls(M, H, KVH, D, Kd, cfg):
    from turingserve_amd import tuner as T

    x, lw, pos, slots, kc, vc = _qkv_problem(M, H, KVH, D, Kd, seed=M + D + Kd)
    cos, sin = rope_tables(D, 1e6, 4096, DEV)
    saved = T.ACTIVE
    try:
        if cfg is not None:                 # route the product through one variant
            table = T.VariantTable()
            table.set("w8a16", ((H + 2 * KVH) * D, Kd, M), {"variant": cfg[0], "splits": cfg[1], "us": 1.0})
            T.set_active(table)
        kc1, vc1 = kc.clone(), vc.clone()
        qkv1 = K.linear_rope_kv_write(x, lw, pos, cos, sin, H, KVH, D, kc1, vc1, slots)
        qkv2 = K.w8a16_linear(x, lw.w, lw.scale, lw.b)
        kc2, vc2 = kc.clone(), vc.clone()
        assert K.rope_kv_write_(qkv2, pos, cos, sin, H, KVH, D, kc2, vc2, slots)
    finally:
        T.set_active(saved)
    torch.cuda.synchronize()
    assert torch.equal(qkv1, qkv2), "qkv differs"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "caches differ"


def test_model_step_with_the_fused_qkv_equals_the_separate_calls():
    """A mixed step (prefill chunks and decode rows) of a random-init model at head_dim 128 with
    W8A16 linears: hidden states and caches equal with and without linear_rope_kv_write."""
    from turingserve_amd import get_ops
    from turingserve_amd.metadata import BatchItem, InputBuilder, SeqState
    from turingserve_amd.qwen2 import Qwen2Config, Qwen2Model, random_weights

    cfg = Qwen2Config(512, 1024, 2, 4, 2, 1000, max_position_embeddings=4096)
    w = random_weights(cfg, DEV, quantization="int8", seed=5)
    fused_ops, plain_ops = get_ops("hip"), get_ops("hip")
    del plain_ops.linear_rope_kv_write
    fused = Qwen2Model(cfg, w, fused_ops, max_model_len=2048)
    plain = Qwen2Model(cfg, w, plain_ops, max_model_len=2048)
    nb = 300
    kv1, kv2 = fused.new_kv_cache(nb), plain.new_kv_cache(nb)
    items, free = [], list(range(1, nb))
    for i in range(10):
        L = 30 + 41 * i
        s = SeqState([(5 * i + 11 * j) % 1000 for j in range(L)])
        s.block_table = [free.pop() for _ in range(-(-L // 16))]
        items.append(s)
    with torch.inference_mode():
        batch = [BatchItem(s, 0, s.token_ids[:-1], "none") for s in items[:6]] + \
                [BatchItem(s, 0, s.token_ids[:20], "none") for s in items[6:]]
        inp = InputBuilder(8192, 64, 32, DEV).build(batch)
        h1 = fused.forward(inp.input_ids, inp.positions, inp.meta, kv1)
        h2 = plain.forward(inp.input_ids, inp.positions, inp.meta, kv2)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2) and torch.equal(kv1, kv2)
