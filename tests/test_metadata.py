"""Host-side metadata (CPU): the vectorised one-copy builder equals a straightforward per-token
restatement of the contract on random plans (the reference's check of its two builders,
tests/correctness/test_paged_engine.py:125-152), slots follow the closed form, and the decode-row
rule of runner/input_builder.py:41-48 holds."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import paged as OP
from turingserve_amd.metadata import BatchItem, InputBuilder, SeqState, num_decode_rows


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


def per_token(items):
    """The contract written out token by token: lists of ids, positions, slots, query_start_loc,
    seq_lens, zero-padded tables, sample rows, and num_decode."""
    ids, pos, slot, qsl, sl, bt, smp = [], [], [], [0], [], [], []
    for it in items:
        table = it.seq.block_table
        for j, tok in enumerate(it.tokens):
            p = it.start + j
            ids.append(tok)
            pos.append(p)
            slot.append(table[p // 16] * 16 + p % 16)
            if it.sample == "all" or (it.sample == "last" and j == len(it.tokens) - 1):
                smp.append(len(ids) - 1)
        qsl.append(len(ids))
        sl.append(it.start + len(it.tokens))
        bt.append(list(table))
    width = max(1, max(len(t) for t in bt))
    bt = [t + [0] * (width - len(t)) for t in bt]
    nd = 0
    while nd < len(items) and len(items[nd].tokens) == 1 and items[nd].sample != "all":
        nd += 1
    return ids, pos, slot, qsl, sl, bt, smp, nd


def test_vectorized_builder_equals_per_token_contract():
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
        ids, pos, slot, qsl, sl, bt, smp, nd = per_token(items)
        b = builder.build(items)
        m = b.meta
        assert b.input_ids.dtype == b.positions.dtype == m.slot_mapping.dtype == torch.int64
        assert m.query_start_loc.dtype == m.seq_lens.dtype == m.block_tables.dtype == torch.int32
        assert b.sample_indices.dtype == torch.int64
        assert b.input_ids.tolist() == ids and b.positions.tolist() == pos
        assert m.slot_mapping.tolist() == slot and m.query_start_loc.tolist() == qsl
        assert m.seq_lens.tolist() == sl and m.block_tables.tolist() == bt
        assert b.sample_indices.tolist() == smp and m.num_decode == nd
        assert m.max_query_len == max(len(it.tokens) for it in items)
        assert m.max_seq_len == max(sl) and m.max_prefill_seq_len == max(sl[nd:], default=0)
        for i, it in enumerate(items):
            want = OP.slot_mapping(it.seq.block_table, np.arange(it.start, it.start + len(it.tokens)))
            assert m.slot_mapping[qsl[i]:qsl[i + 1]].tolist() == want.tolist()
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


def test_pack_step_upload_expands_to_the_per_token_contract():
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
        want = per_token(items)
        width = len(want[5][0])
        assert _expand(words, len(items), T, width) == want[:7] and S == len(want[6])
        for it in items:
            blocks.release(it.seq)


def test_position_past_the_table_is_an_error():
    b = InputBuilder(64, 4, 8, "cpu")
    s = SeqState(list(range(40)), [7])
    with pytest.raises(ValueError, match="past its 1-block table"):
        b.build([BatchItem(s, 14, list(range(14, 18)), "all")])


def test_one_upload_holds_every_array():
    """Every tensor of the step is a view of the builder's one device arena."""
    b = InputBuilder(64, 4, 8, "cpu")
    s = SeqState(list(range(20)), [3, 4])
    inp = b.build([BatchItem(s, 0, list(range(20)), "last")])
    base = b._arena.untyped_storage().data_ptr()
    for t in (inp.input_ids, inp.positions, inp.sample_indices, inp.meta.slot_mapping,
              inp.meta.query_start_loc, inp.meta.seq_lens, inp.meta.block_tables):
        assert t.untyped_storage().data_ptr() == base
    assert inp.meta.slot_mapping.tolist() == [3 * 16 + p for p in range(16)] + [4 * 16 + p for p in range(4)]
