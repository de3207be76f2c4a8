"""Sequences that share full prefix blocks (needs an MI355X).

The reference's prefix cache shares full, immutable blocks between sequences
(kv/prefix_cache.py:1-4): their block tables then name the same physical blocks for the shared
prefix, and only the blocks after it are a sequence's own. These tests build such tables (several
sequences over one run of shared blocks, each continuing in blocks of its own, the new tokens'
slots in those) and run the HIP path over them against the oracle (ops/reference.py:60-111):

* decode attention alone (the automatic policy, v2 and a fixed 256-token v3 grid);
* the fused rope + kv_write + decode launch, bit-equal to rope_kv_write followed by
  paged_attention, its attention against the oracle on the caches it wrote, and the shared
  blocks untouched;
* a mixed step: those decode rows beside a prefill chunk of a prompt whose prefix is the same
  cached run of shared blocks (a prefix-cache hit), through one paged_attention call.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from turingserve_amd import hip_ops as K
from turingserve_amd.metadata import AttentionMetadata

from .test_decode_kv_write_gpu import rope_tables
from .test_kernels_gpu import DEV, assert_attn, oracle_attn

pytestmark = pytest.mark.gpu
H, KVH, D = 12, 2, 128


def shared_layout(prefix_blocks, tails, seed, extra=()):
    """Block tables for len(tails) sequences that share `prefix_blocks` full blocks, sequence i
    continuing with tails[i] tokens in blocks of its own; `extra` adds sequences (prompt tails)
    after them in the same way. Returns (kc, vc, seq_lens, bt, shared block ids)."""
    g = torch.Generator().manual_seed(seed)
    tails = list(tails) + list(extra)
    own = [-(-t // 16) for t in tails]
    total = 1 + prefix_blocks + sum(own)
    perm = torch.randperm(total - 1, generator=g) + 1       # block 0 stays unused
    shared = perm[:prefix_blocks]
    kc = torch.randn(total, KVH, 16, D, generator=g).half()
    vc = torch.randn(total, KVH, 16, D, generator=g).half()
    width = prefix_blocks + max(own)
    bt = torch.zeros(len(tails), width, dtype=torch.int32)
    off = prefix_blocks
    for i, nb in enumerate(own):
        bt[i, :prefix_blocks] = shared.int()
        bt[i, prefix_blocks:prefix_blocks + nb] = perm[off:off + nb].int()
        off += nb
    sl = torch.tensor([prefix_blocks * 16 + t for t in tails], dtype=torch.int32)
    return kc, vc, sl, bt, shared


def decode_meta(sl, bt, slots=None):
    n = sl.shape[0]
    qsl = torch.arange(n + 1, dtype=torch.int32)
    sm = slots if slots is not None else torch.zeros(n, dtype=torch.int64)
    return AttentionMetadata(qsl.to(DEV), sl.to(DEV), bt.to(DEV), sm.to(DEV), n, 1, int(sl.max()))


@pytest.mark.parametrize("prefix_blocks,tails", [
    (8, [1, 5, 16, 17, 40, 200]),            # short tails, one exactly a block
    (64, [3, 100, 333, 1000]),               # a 1024-token shared prefix, splits over it
    (1, [15, 2, 64]),
])
@pytest.mark.parametrize("version,partition", [(None, None), ("v2", None), ("v3", 256)])
def test_decode_over_shared_prefix_blocks(prefix_blocks, tails, version, partition):
    kc, vc, sl, bt, _ = shared_layout(prefix_blocks, tails, seed=prefix_blocks + len(tails))
    g = torch.Generator().manual_seed(5)
    q = torch.randn(len(tails), H, D, generator=g).half()
    meta = decode_meta(sl, bt)
    out = K.paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), meta, D ** -0.5,
                            decode_version=version, partition=partition)
    ref = oracle_attn(q, kc, vc, meta.query_start_loc.cpu(), sl, bt, D ** -0.5)
    assert_attn(out, ref, f"shared prefix {prefix_blocks} blocks, {version}/{partition}")


@pytest.mark.parametrize("prefix_blocks,tails", [(8, [1, 5, 17, 40]), (64, [3, 100, 333])])
def test_fused_rope_write_decode_over_shared_prefix_blocks(prefix_blocks, tails):
    kc, vc, sl, bt, shared = shared_layout(prefix_blocks, tails, seed=11 + prefix_blocks)
    n = len(tails)
    # the step's new token of sequence i sits at position seq_len - 1, in a block of its own
    pos = sl.long() - 1
    slots = torch.tensor([int(bt[i, int(pos[i]) // 16]) * 16 + int(pos[i]) % 16 for i in range(n)],
                         dtype=torch.int64)
    meta = decode_meta(sl, bt, slots)
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(n, (H + 2 * KVH) * D, generator=g).half()
    cos, sin = rope_tables(D, int(sl.max()) + 16)
    qkv1, kc1, vc1 = qkv.to(DEV), kc.to(DEV), vc.to(DEV)
    assert K.rope_kv_write_(qkv1, pos.to(DEV), cos, sin, H, KVH, D, kc1, vc1, meta.slot_mapping)
    q1 = qkv1[:, :H * D].view(-1, H, D)
    sep = K.paged_attention(q1, kc1, vc1, meta, D ** -0.5)
    qkv2, kc2, vc2 = qkv.to(DEV), kc.to(DEV), vc.to(DEV)
    out = K.decode_rope_kv_write_attention(qkv2, pos.to(DEV), cos, sin, H, KVH, D, kc2, vc2, meta,
                                           D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "caches differ"
    assert torch.equal(out, sep), "fused output differs from rope_kv_write + paged_attention"
    sh = shared.long().to(DEV)
    assert torch.equal(kc2[sh], kc.to(DEV)[sh]) and torch.equal(vc2[sh], vc.to(DEV)[sh]), \
        "a shared prefix block was written"
    ref = oracle_attn(q1.cpu(), kc2.cpu(), vc2.cpu(), meta.query_start_loc.cpu(), sl, bt,
                      D ** -0.5)
    assert_attn(out, ref, "fused, shared prefix")


@pytest.mark.parametrize("prefix_blocks,chunk", [(8, 300), (64, 512)])
def test_mixed_step_with_a_prefix_cache_hit(prefix_blocks, chunk):
    """Decode rows over the shared prefix and, in the same paged_attention call, the prefill
    chunk of a new prompt whose first prefix_blocks blocks are that cached run (its chunk's
    queries start right after it)."""
    tails = [1, 7, 33, 200, 64]
    kc, vc, sl, bt, _ = shared_layout(prefix_blocks, tails, seed=21 + chunk, extra=(chunk,))
    n = len(tails)
    g = torch.Generator().manual_seed(9)
    q = torch.randn(n + chunk, H, D, generator=g).half()
    q_lens = [1] * n + [chunk]
    qsl = torch.tensor([0] + np.cumsum(q_lens).tolist(), dtype=torch.int32)
    meta = AttentionMetadata(qsl.to(DEV), sl.to(DEV), bt.to(DEV),
                             torch.zeros(n + chunk, dtype=torch.int64, device=DEV), n, chunk,
                             int(sl.max()))
    out = K.paged_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), meta, D ** -0.5)
    ref = oracle_attn(q, kc, vc, qsl, sl, bt, D ** -0.5)
    assert_attn(out, ref, f"mixed step, prefix-cache hit of {prefix_blocks} blocks")
