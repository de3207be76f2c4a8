"""kv_write fused into the decode attention launch (ts_decode_attention_kv_write) against the
two separate calls and the oracle (needs an MI355X).

A pure-decode layer step is kv_write of the new K/V rows (ops/triton_kv_write.py:28-35) and
then paged attention over every cached token including them (ops/triton_ops.py:60-71). The
fused entry point must leave bit-identical caches and return bit-identical outputs to
K.kv_write followed by K.paged_attention with the same decode policy (the attention arithmetic
is the same kernel's), and match the oracle (ops/reference.py:50-57 then :94-111) with the
attention criterion of the other kernel tests. Cases where the write cannot be fused (v1,
more than 16 query heads per KV head) take the two-launch route inside the library and must
give the same results.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged as OP
from turingserve_amd import hip_ops as K
from turingserve_amd import synth
from turingserve_amd.metadata import AttentionMetadata

from .test_kernels_gpu import DEV, assert_attn, make_paged

pytestmark = pytest.mark.gpu


def decode_step(ctx, H, KVH, D, seed, pad=()):
    """A decode step: sequence i has ctx[i] tokens after it (its new token at position
    ctx[i] - 1, slot from its block table); rows in `pad` are graph padding (seq_len 0,
    slot -1). q, k, v are strided views of one qkv buffer, as the model produces them."""
    g = torch.Generator().manual_seed(seed + 1000)
    ctx = list(ctx)
    for i in pad:
        ctx[i] = 0
    _, kc, vc, qsl, sl, bt = make_paged(ctx, H, KVH, D, seed=seed)
    B = len(ctx)
    qkv = torch.randn(B, (H + 2 * KVH) * D, generator=g).half()
    slots = torch.tensor([int(bt[i, (c - 1) // 16]) * 16 + (c - 1) % 16 if c > 0 else -1
                          for i, c in enumerate(ctx)], dtype=torch.int64)
    return qkv, kc, vc, qsl, sl, bt, slots


def views(qkv, H, KVH, D):
    B = qkv.shape[0]
    q = qkv[:, :H * D].view(B, H, D)
    k = qkv[:, H * D:(H + KVH) * D].view(B, KVH, D)
    v = qkv[:, (H + KVH) * D:].view(B, KVH, D)
    return q, k, v


def meta_for(qsl, sl, bt, slots):
    B = sl.shape[0]
    return AttentionMetadata(qsl.to(DEV), sl.to(DEV), bt.to(DEV), slots.to(DEV), B, 1,
                             max(1, int(sl.max())))


def run_both(case, H, KVH, D, version, partition):
    qkv, kc, vc, qsl, sl, bt, slots = case
    meta = meta_for(qsl, sl, bt, slots)
    q, k, v = views(qkv.to(DEV), H, KVH, D)
    scale = D ** -0.5
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    K.kv_write(k, v, kc1, vc1, meta.slot_mapping)
    ref = K.paged_attention(q, kc1, vc1, meta, scale, decode_version=version, partition=partition)
    kc2, vc2 = kc.to(DEV), vc.to(DEV)
    out = K.decode_kv_write_attention(q, k, v, kc2, vc2, meta, scale, decode_version=version,
                                      partition=partition)
    torch.cuda.synchronize()
    return out, ref, (kc1, vc1), (kc2, vc2)


@pytest.mark.parametrize("H,KVH,D,version,partition", [
    (12, 2, 128, None, None),       # config 2 heads: own-length split-K, fused
    (12, 2, 128, "v2", None),       # one workgroup per (sequence, KV head), fused
    (12, 2, 128, "v3", 512),        # the reference's fixed partition grid, fused
    (12, 2, 128, "v1", None),       # no MFMA kernel: kv_write's own launch first
    (14, 2, 64, None, None),        # Qwen2.5-0.5B heads
    (32, 1, 128, None, None),       # 32 query heads per KV head: two head groups, two launches
    (4, 4, 16, None, None),         # smallest head_dim, no GQA
])
def test_fused_matches_separate_calls_and_oracle(H, KVH, D, version, partition):
    g = torch.Generator().manual_seed(H * 100 + D)
    ctx = synth.log_uniform_ints(64, 17, 4096, g)
    ctx[3], ctx[7], ctx[11] = 1, 16, 33       # a one-token context and block boundaries
    case = decode_step(ctx, H, KVH, D, seed=H + D)
    out, ref, (kc1, vc1), (kc2, vc2) = run_both(case, H, KVH, D, version, partition)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "caches differ"
    assert torch.equal(out, ref), "fused output differs from kv_write + paged_attention"
    qkv, kc, vc, qsl, sl, bt, slots = case
    q, k, v = views(qkv, H, KVH, D)
    kcn, vcn = kc.numpy().copy(), vc.numpy().copy()
    OP.kv_write(k.numpy(), v.numpy(), kcn, vcn, slots.numpy())
    oref = OP.paged_attention(q.numpy(), kcn, vcn, qsl.numpy(), sl.numpy(), bt.numpy(), D ** -0.5)
    assert_attn(out, oref, "fused decode")


def test_fused_padding_rows():
    """Graph padding rows (seq_len 0, slot -1) are written as zeros and touch no cache row."""
    H, KVH, D = 12, 2, 128
    g = torch.Generator().manual_seed(5)
    ctx = synth.log_uniform_ints(48, 100, 3000, g)
    case = decode_step(ctx, H, KVH, D, seed=5, pad=(0, 17, 47))
    out, ref, (kc1, vc1), (kc2, vc2) = run_both(case, H, KVH, D, None, None)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(out, ref)
    for i in (0, 17, 47):
        assert torch.equal(out[i], torch.zeros_like(out[i]))


def test_fused_config2_graph_replays():
    """The config 2 step captured in a graph: every replay (with eager work between them)
    equals the eager fused call and the two-call step."""
    st = synth.config2(seed=3)
    qkv = st.qkv.to(DEV)
    q, k, v = st.views(qkv)
    meta = st.meta(DEV)
    meta.in_graph = True
    scale = st.D ** -0.5
    kc, vc = st.k_cache.to(DEV), st.v_cache.to(DEV)
    K.kv_write(k, v, kc, vc, meta.slot_mapping)
    ref = K.paged_attention(q, kc, vc, meta, scale)
    kc2, vc2 = st.k_cache.to(DEV), st.v_cache.to(DEV)
    eager = K.decode_kv_write_attention(q, k, v, kc2, vc2, meta, scale)
    assert torch.equal(eager, ref) and torch.equal(kc2, kc) and torch.equal(vc2, vc)
    outs = []
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs.append(K.decode_kv_write_attention(q, k, v, kc2, vc2, meta, scale))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[0], ref)
        scratch = torch.randn(1 << 20, device=DEV).sum()     # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)


# ------------------------------------------------------------------------------------------
# RoPE fused as well (ts_decode_rope_kv_write_attention)
# ------------------------------------------------------------------------------------------
def rope_tables(D, max_len, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cos(ang).float().to(DEV), torch.sin(ang).float().to(DEV)


@pytest.mark.parametrize("H,KVH,D,version,positions", [
    (12, 2, 128, None, "last"),     # Qwen2.5-1.5B heads, split-K, fused
    (12, 2, 128, "v2", "last"),
    (14, 2, 64, None, "last"),      # Qwen2.5-0.5B heads, fused
    (8, 8, 256, None, "last"),      # head_dim 256, fused
    (12, 2, 128, None, "wild"),     # positions not tied to seq_lens, some out of the table
    (12, 2, 128, "v1", "last"),     # v1: rope_kv_write's own launch first
    (32, 1, 128, None, "last"),     # two head groups per KV head: separate launches
    (4, 2, 32, None, "last"),       # head_dim 32: rotation pairs span lanes, separate launches
])
def test_rope_fused_matches_separate_calls(H, KVH, D, version, positions):
    g = torch.Generator().manual_seed(H * 10 + D)
    ctx = synth.log_uniform_ints(48, 2, 3000, g)
    ctx[5] = 1
    case = decode_step(ctx, H, KVH, D, seed=H + D + 7, pad=(9,))
    qkv, kc, vc, qsl, sl, bt, slots = case
    meta = meta_for(qsl, sl, bt, slots)
    cos, sin = rope_tables(D, 3000)
    if positions == "last":
        pos = (sl.long() - 1).clamp(min=0)
    else:
        pos = torch.randint(-5, 3100, (len(ctx),), generator=g)
    pos = pos.to(DEV)
    scale = D ** -0.5
    # separate calls: rope + kv_write in one pass, then attention over the rotated q
    qkv1 = qkv.to(DEV)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    assert K.rope_kv_write_(qkv1, pos, cos, sin, H, KVH, D, kc1, vc1, meta.slot_mapping)
    q1 = qkv1[:, :H * D].view(-1, H, D)
    ref = K.paged_attention(q1, kc1, vc1, meta, scale, decode_version=version)
    qkv2 = qkv.to(DEV)
    kc2, vc2 = kc.to(DEV), vc.to(DEV)
    out = K.decode_rope_kv_write_attention(qkv2, pos, cos, sin, H, KVH, D, kc2, vc2, meta, scale,
                                           decode_version=version)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "caches differ"
    assert torch.equal(out, ref), "fused output differs from rope_kv_write + paged_attention"
    assert torch.equal(out[9], torch.zeros_like(out[9]))


def test_rope_fused_model_decode_step():
    """A random-init model with head_dim 128 (and 64): a pure-decode step takes the fused launch
    in every layer and must give the hidden states and caches of the separate calls."""
    from turingserve_amd import get_ops
    from turingserve_amd.metadata import BatchItem, InputBuilder, SeqState
    from turingserve_amd.qwen2 import Qwen2Config, Qwen2Model, random_weights

    for cfg in (Qwen2Config(512, 1024, 2, 4, 2, 1000, max_position_embeddings=4096),
                Qwen2Config(448, 896, 2, 7, 1, 1000, max_position_embeddings=4096)):
        w = random_weights(cfg, DEV, seed=3)
        fused_ops = get_ops("hip")
        plain_ops = get_ops("hip")
        del plain_ops.decode_rope_kv_write_attention
        fused = Qwen2Model(cfg, w, fused_ops, max_model_len=2048)
        plain = Qwen2Model(cfg, w, plain_ops, max_model_len=2048)
        nb = 400
        kv1, kv2 = fused.new_kv_cache(nb), plain.new_kv_cache(nb)
        items, free = [], list(range(1, nb))
        for i in range(12):
            L = 20 + 37 * i
            s = SeqState([(7 * i + 3 * j) % 1000 for j in range(L)])
            s.block_table = [free.pop() for _ in range(-(-L // 16))]
            items.append(s)
        with torch.inference_mode():
            pre = InputBuilder(8192, 64, 32, DEV).build(
                [BatchItem(s, 0, s.token_ids[:-1], "none") for s in items])
            fused.forward(pre.input_ids, pre.positions, pre.meta, kv1)
            plain.forward(pre.input_ids, pre.positions, pre.meta, kv2)
            assert torch.equal(kv1, kv2)
            dec = InputBuilder(256, 64, 32, DEV).build(
                [BatchItem(s, len(s.token_ids) - 1, [s.token_ids[-1]], "last") for s in items])
            h1 = fused.forward(dec.input_ids, dec.positions, dec.meta, kv1)
            h2 = plain.forward(dec.input_ids, dec.positions, dec.meta, kv2)
        torch.cuda.synchronize()
        assert torch.equal(h1, h2) and torch.equal(kv1, kv2)


@pytest.mark.parametrize("version,partition,rope", [(None, None, False), ("v2", None, False),
                                                    ("v3", 512, False), (None, None, True)])
def test_fused_write_with_a_foreign_slot_gives_nan_not_a_race(version, partition, rope):
    """The fusion's precondition is that slot_mapping[i] is the slot of position seq_lens[i] - 1.
    A row whose slot points elsewhere (into another sequence's block, which another workgroup
    may be reading) is not written; that sequence's output is NaN, every other row and the rest
    of the cache are exactly those of the separate calls."""
    H, KVH, D = 12, 2, 128
    ctx = [700, 33, 1500, 64, 900]
    qkv, kc, vc, qsl, sl, bt, slots = decode_step(ctx, H, KVH, D, seed=5)
    bad = 2
    slots = slots.clone()
    slots[bad] = int(bt[0, 3]) * 16 + 5                   # a slot in sequence 0's fourth block
    meta = meta_for(qsl, sl, bt, slots)
    scale = D ** -0.5
    kc2, vc2 = kc.to(DEV), vc.to(DEV)
    if rope:
        from turingserve_amd.qwen2 import rope_tables

        cos, sin = rope_tables(D, 1e6, 4096, DEV)
        pos = (sl.to(DEV).long() - 1).clamp_min(0)
        out = K.decode_rope_kv_write_attention(qkv.to(DEV).contiguous(), pos, cos, sin, H, KVH,
                                               D, kc2, vc2, meta, scale,
                                               decode_version=version, partition=partition)
    else:
        q, k, v = views(qkv.to(DEV), H, KVH, D)
        out = K.decode_kv_write_attention(q, k, v, kc2, vc2, meta, scale, decode_version=version,
                                          partition=partition)
    torch.cuda.synchronize()
    o = out.float().cpu()
    assert bool(torch.isnan(o[bad]).all())
    assert not bool(torch.isnan(o[[i for i in range(len(ctx)) if i != bad]]).any())
    # the foreign slot was not written
    blk, off = int(slots[bad]) // 16, int(slots[bad]) % 16
    assert torch.equal(kc2[blk, :, off].cpu(), kc[blk, :, off])
    assert torch.equal(vc2[blk, :, off].cpu(), vc[blk, :, off])
