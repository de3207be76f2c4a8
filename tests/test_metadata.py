"""Host-side metadata (CPU): the vectorised builder equals the straightforward one on random plans
(the reference's tests/correctness/test_paged_engine.py:125-152), slots follow the closed form, and
the decode-row rule of runner/input_builder.py:41-48 holds."""

from __future__ import annotations

import random

import numpy as np
import torch

from oracle import paged as OP
from turingserve_amd.metadata import BatchItem, InputBuilder, SeqState, build_simple, num_decode_rows


class Blocks:
    """Minimal allocator: block 0 is the null block, ids handed out shuffled."""

    def __init__(self, n: int, seed: int = 0) -> None:
        self.free = list(range(1, n))
        random.Random(seed).shuffle(self.free)

    def grow(self, seq: SeqState, tokens: int) -> None:
        while len(seq.block_table) * 16 < tokens:
            seq.block_table.append(self.free.pop())

    def release(self, seq: SeqState) -> None:
        self.free.extend(seq.block_table)
        seq.block_table = []


def test_vectorized_builder_equals_simple_builder():
    rng = random.Random(0)
    builder = InputBuilder(2048, 16, 128, "cpu")
    blocks = Blocks(400)
    for _ in range(200):
        items = []
        for _i in range(rng.randint(1, 8)):
            n_prompt = rng.randint(1, 120)
            s = SeqState([rng.randrange(1000) for _ in range(n_prompt)])
            start = rng.randint(0, n_prompt - 1)
            n = rng.randint(1, n_prompt - start)
            blocks.grow(s, start + n)
            items.append(BatchItem(s, start, s.token_ids[start:start + n],
                                   rng.choice(["last", "none", "all"])))
        items.sort(key=lambda it: len(it.tokens) != 1)
        a, b = build_simple(items, "cpu"), builder.build(items)
        assert torch.equal(a.input_ids, b.input_ids) and torch.equal(a.positions, b.positions)
        assert torch.equal(a.meta.slot_mapping, b.meta.slot_mapping)
        assert torch.equal(a.meta.query_start_loc, b.meta.query_start_loc)
        assert torch.equal(a.meta.seq_lens, b.meta.seq_lens)
        w = a.meta.block_tables.shape[1]
        assert torch.equal(a.meta.block_tables, b.meta.block_tables[:, :w])
        assert torch.equal(a.sample_indices, b.sample_indices)
        assert a.meta.num_decode == b.meta.num_decode
        assert a.meta.max_query_len == b.meta.max_query_len
        assert a.meta.max_seq_len == b.meta.max_seq_len
        for it in items:
            want = OP.slot_mapping(it.seq.block_table, np.arange(it.start, it.start + len(it.tokens)))
            lo = int(a.meta.query_start_loc[items.index(it)])
            assert a.meta.slot_mapping[lo:lo + len(it.tokens)].tolist() == want.tolist()
            blocks.release(it.seq)


def test_num_decode_rule():
    s = SeqState([1, 2, 3], [1])
    items = [BatchItem(s, 2, [3]), BatchItem(s, 2, [3], "none"), BatchItem(s, 0, [1, 2]),
             BatchItem(s, 2, [3])]
    assert num_decode_rows(items) == 2
    assert num_decode_rows([BatchItem(s, 2, [3], "all")]) == 0


def test_stale_block_table_rows_are_cleared():
    b = InputBuilder(64, 4, 8, "cpu")
    long_seq = SeqState(list(range(100)), [5, 6, 7, 8, 9, 10, 11])
    b.build([BatchItem(long_seq, 99, [99])])
    short = SeqState([1], [3])
    two = SeqState(list(range(20)), [1, 2])
    m = b.build([BatchItem(short, 0, [1]), BatchItem(two, 19, [19])]).meta
    assert m.block_tables.tolist() == [[3, 0], [1, 2]]


def _expand(words: np.ndarray, B: int, T: int, width: int):
    """Straightforward expansion of pack_step's upload, following ts_step_metadata's contract."""
    desc = words[:5 * B].reshape(B, 5).astype(np.int64)
    toks = words[5 * B:5 * B + T].astype(np.int64)
    blocks = words[5 * B + T:].astype(np.int64)
    ids, pos, slot, qsl, sl, bt, smp = [], [], [], [0], [], [], []
    off = 0
    for start, n, mode, t_off, t_len in desc:
        table = blocks[t_off:t_off + t_len]
        for t in range(n):
            p = start + t
            ids.append(toks[off + t])
            pos.append(p)
            slot.append(table[p // 16] * 16 + p % 16 if p // 16 < t_len else -1)
        if mode == 1 and n > 0:
            smp.append(off + n - 1)
        elif mode == 2:
            smp += list(range(off, off + n))
        off += n
        qsl.append(off)
        sl.append(start + n)
        bt.append(list(table) + [0] * (width - t_len))
    return ids, pos, slot, qsl, sl, bt, smp


def test_pack_step_upload_expands_to_the_simple_builder():
    from turingserve_amd.metadata import pack_step

    rng = random.Random(1)
    blocks = Blocks(400, seed=1)
    for _ in range(100):
        items = []
        for _i in range(rng.randint(1, 8)):
            n_prompt = rng.randint(1, 120)
            s = SeqState([rng.randrange(150000) for _ in range(n_prompt)])
            start = rng.randint(0, n_prompt - 1)
            n = rng.randint(1, n_prompt - start)
            blocks.grow(s, start + n + rng.randint(0, 40))      # tables may run ahead
            items.append(BatchItem(s, start, s.token_ids[start:start + n],
                                   rng.choice(["last", "none", "all"])))
        items.sort(key=lambda it: len(it.tokens) != 1)
        words, T, NB, S = pack_step(items)
        assert words.dtype == np.int32 and words.size == 5 * len(items) + T + NB
        a = build_simple(items, "cpu")
        width = a.meta.block_tables.shape[1]
        ids, pos, slot, qsl, sl, bt, smp = _expand(words, len(items), T, width)
        assert ids == a.input_ids.tolist() and pos == a.positions.tolist()
        assert slot == a.meta.slot_mapping.tolist() and qsl == a.meta.query_start_loc.tolist()
        assert sl == a.meta.seq_lens.tolist() and bt == a.meta.block_tables.tolist()
        assert smp == a.sample_indices.tolist() and S == len(smp)
        for it in items:
            blocks.release(it.seq)
