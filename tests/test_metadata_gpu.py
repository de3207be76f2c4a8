"""Device-side step metadata (ts_step_metadata through DeviceInputBuilder) on the GPU: equal, row
for row, to the host builder (InputBuilder, pinned on the CPU against a per-token restatement of
the contract of runner/input_builder.py:41-150), including the padding rows a captured decode
graph expects (runner/cuda_graphs.py:62-78), and an engine driven by it generates the same
tokens."""

from __future__ import annotations

import random

import pytest
import torch

from tests.test_metadata import Blocks
from turingserve_amd.metadata import BatchItem, DeviceInputBuilder, InputBuilder, SeqState

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _random_items(rng, blocks, k):
    items = []
    for _ in range(k):
        n_prompt = rng.randint(1, 300)
        s = SeqState([rng.randrange(150000) for _ in range(n_prompt)])
        start = rng.randint(0, n_prompt - 1)
        n = rng.randint(1, min(64, n_prompt - start))
        if rng.random() < 0.5:
            start, n = n_prompt - 1, 1                       # a decode row
        blocks.grow(s, start + n + rng.randint(0, 20))
        items.append(BatchItem(s, start, s.token_ids[start:start + n],
                               rng.choice(["last", "last", "none", "all"])))
    items.sort(key=lambda it: len(it.tokens) != 1)
    return items


def test_device_builder_equals_host_builder():
    rng = random.Random(0)
    blocks = Blocks(3000, seed=2)
    host = InputBuilder(4096, 64, 64, DEV)
    dev = DeviceInputBuilder(4096, 64, 64, DEV)
    for k in [1, 2, 7, 33, 64] * 6:
        items = _random_items(rng, blocks, k)
        a, b = host.build(items), dev.build(items)
        torch.cuda.synchronize()
        for x, y in ((a.input_ids, b.input_ids), (a.positions, b.positions),
                     (a.meta.slot_mapping, b.meta.slot_mapping),
                     (a.meta.query_start_loc, b.meta.query_start_loc),
                     (a.meta.seq_lens, b.meta.seq_lens), (a.meta.block_tables, b.meta.block_tables),
                     (a.sample_indices, b.sample_indices)):
            assert x.dtype == y.dtype and torch.equal(x, y)
        assert (a.meta.num_decode, a.meta.max_query_len, a.meta.max_seq_len,
                a.meta.max_prefill_seq_len) == (b.meta.num_decode, b.meta.max_query_len,
                                                b.meta.max_seq_len, b.meta.max_prefill_seq_len)
        for it in items:
            blocks.release(it.seq)


def test_slots_past_the_table_are_padding():
    dev = DeviceInputBuilder(64, 4, 8, DEV)
    s = SeqState(list(range(40)), [7])                   # a table of one block for 40 tokens
    inp = dev.build([BatchItem(s, 14, list(range(14, 18)), "all")])
    assert inp.meta.slot_mapping.tolist() == [7 * 16 + 14, 7 * 16 + 15, -1, -1]
    assert inp.sample_indices.tolist() == [0, 1, 2, 3]


def test_build_into_pads_like_graph_replay():
    dev = DeviceInputBuilder(64, 8, 16, DEV)
    B, n = 8, 3
    ids = torch.full((B,), 123, dtype=torch.int64, device=DEV)
    pos, slot = ids.clone(), ids.clone()
    qsl = torch.full((B + 1,), 77, dtype=torch.int32, device=DEV)
    sl = torch.full((B,), 55, dtype=torch.int32, device=DEV)
    bt = torch.full((B, 16), 9, dtype=torch.int32, device=DEV)
    seqs = [SeqState(list(range(20 + 17 * i)), list(range(1 + 5 * i, 3 + 6 * i))) for i in range(n)]
    items = [BatchItem(s, len(s.token_ids) - 1, [s.token_ids[-1]]) for s in seqs]
    dev.build_into(items, B, ids, pos, slot, qsl, sl, bt)
    ref = InputBuilder(64, 8, 16, DEV).build(items)
    torch.cuda.synchronize()
    assert ids[:n].tolist() == ref.input_ids.tolist() and ids[n:].tolist() == [0] * (B - n)
    assert pos[:n].tolist() == ref.positions.tolist() and pos[n:].tolist() == [0] * (B - n)
    assert slot[:n].tolist() == ref.meta.slot_mapping.tolist() and slot[n:].tolist() == [-1] * (B - n)
    assert sl[:n].tolist() == ref.meta.seq_lens.tolist() and sl[n:].tolist() == [0] * (B - n)
    assert qsl.tolist() == list(range(B + 1))
    w = ref.meta.block_tables.shape[1]
    assert torch.equal(bt[:n, :w], ref.meta.block_tables)
    assert int(bt[:n, w:].abs().sum()) == 0 and int(bt[n:].abs().sum()) == 0


def test_engine_with_device_metadata_generates_the_same_tokens():
    from turingserve_amd import get_ops
    from turingserve_amd.engine import GreedyEngine
    from turingserve_amd.qwen2 import TINY_G2, Qwen2Model, random_weights

    w = random_weights(TINY_G2, DEV, seed=1)
    model = Qwen2Model(TINY_G2, w, get_ops("hip"))
    rng = random.Random(3)
    prompts = [[rng.randrange(1000) for _ in range(rng.randint(3, 40))] for _ in range(6)]
    kw = dict(max_num_batched_tokens=48, max_num_seqs=8, graph_sizes=(1, 2, 4, 8))
    a = GreedyEngine(model, 300, **kw)
    b = GreedyEngine(model, 300, device_metadata=True, **kw)
    out_a, out_b = a.generate(prompts, 12), b.generate(prompts, 12)
    assert out_a == out_b
    assert b.graph_steps > 0 and b.graph_steps == a.graph_steps
