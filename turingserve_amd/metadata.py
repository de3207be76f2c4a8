"""Attention metadata of one flat ragged batch, and the host builders that produce it.

Restates the reference's kernel input contract (runner/attention_metadata.py:10-27) and its two
builders (runner/input_builder.py:41-150): rows [0, num_decode) are decodes with one query token
each (q row index == sequence index), then prefill chunks; ``seq_lens`` is the context length
after this step; ``slot_mapping[t] = table[pos // 16] * 16 + pos % 16`` (-1 = padding row);
block-table rows are padded with block 0, the null block.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

BLOCK_SIZE = 16


@dataclass
class AttentionMetadata:
    query_start_loc: torch.Tensor     # [B+1] int32 (cu_seqlens)
    seq_lens: torch.Tensor            # [B]   int32, context length AFTER this step
    block_tables: torch.Tensor        # [B, max_blocks_per_seq] int32, padded with 0
    slot_mapping: torch.Tensor        # [T] int64, -1 = padding
    num_decode: int                   # first num_decode rows have query_len 1
    max_query_len: int
    max_seq_len: int
    in_graph: bool = False            # set while capturing / replaying a hipGraph


@dataclass
class ModelInput:
    input_ids: torch.Tensor           # [T] int64
    positions: torch.Tensor           # [T] int64
    meta: AttentionMetadata
    sample_indices: torch.Tensor      # [S] int64, rows turned into logits


@dataclass
class SeqState:
    """What the builders need from a sequence: its token ids and its KV block table."""

    token_ids: list[int]
    block_table: list[int] = field(default_factory=list)


@dataclass
class BatchItem:
    """``tokens`` occupy positions start .. start+len-1 of ``seq``; sample is 'last' (one logits
    row), 'all' (a row per token) or 'none' (runner/input_builder.py:20-29)."""

    seq: SeqState
    start: int
    tokens: list[int]
    sample: str = "last"


def num_decode_rows(items: list[BatchItem]) -> int:
    """Leading items with exactly one token that do not sample every row
    (runner/input_builder.py:41-48)."""
    n = 0
    for it in items:
        if len(it.tokens) == 1 and it.sample != "all":
            n += 1
        else:
            break
    return n


def build_simple(items: list[BatchItem], device) -> ModelInput:
    """Straightforward per-token builder (runner/input_builder.py:51-78)."""
    ids, pos, slots, qsl, seq_lens, tables, sample = [], [], [], [0], [], [], []
    for it in items:
        n = len(it.tokens)
        p = list(range(it.start, it.start + n))
        bt = it.seq.block_table
        ids += it.tokens
        pos += p
        slots += [bt[x // BLOCK_SIZE] * BLOCK_SIZE + x % BLOCK_SIZE for x in p]
        qsl.append(qsl[-1] + n)
        seq_lens.append(it.start + n)
        tables.append(list(bt))
        if it.sample == "last":
            sample.append(qsl[-1] - 1)
        elif it.sample == "all":
            sample += list(range(qsl[-2], qsl[-1]))
    width = max(1, max(len(t) for t in tables))
    tables = [t + [0] * (width - len(t)) for t in tables]
    meta = AttentionMetadata(
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=device),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=device),
        block_tables=torch.tensor(tables, dtype=torch.int32, device=device),
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        num_decode=num_decode_rows(items), max_query_len=max(len(i.tokens) for i in items),
        max_seq_len=max(seq_lens))
    return ModelInput(torch.tensor(ids, dtype=torch.int64, device=device),
                      torch.tensor(pos, dtype=torch.int64, device=device), meta,
                      torch.tensor(sample, dtype=torch.int64, device=device))


class InputBuilder:
    """Vectorised builder with persistent host (pinned on a GPU) and device buffers
    (runner/input_builder.py:81-150). The host buffers are rewritten only after the previous
    step's sampler synchronisation, so no in-flight copy can still be reading them."""

    def __init__(self, max_tokens: int, max_seqs: int, max_blocks_per_seq: int, device) -> None:
        self.device = torch.device(device)
        pin = self.device.type == "cuda"

        def host(shape, dtype):
            return torch.zeros(shape, dtype=dtype, pin_memory=pin)

        def dev(shape, dtype):
            return torch.zeros(shape, dtype=dtype, device=self.device)

        self.max_tokens, self.max_seqs, self.max_blocks = max_tokens, max_seqs, max_blocks_per_seq
        i32, i64 = torch.int32, torch.int64
        self.h_ids, self.d_ids = host(max_tokens, i64), dev(max_tokens, i64)
        self.h_pos, self.d_pos = host(max_tokens, i64), dev(max_tokens, i64)
        self.h_slot, self.d_slot = host(max_tokens, i64), dev(max_tokens, i64)
        self.h_sample, self.d_sample = host(max_tokens, i64), dev(max_tokens, i64)
        self.h_qsl, self.d_qsl = host(max_seqs + 1, i32), dev(max_seqs + 1, i32)
        self.h_sl, self.d_sl = host(max_seqs, i32), dev(max_seqs, i32)
        self.h_bt = host((max_seqs, max_blocks_per_seq), i32)
        self.d_bt = dev((max_seqs, max_blocks_per_seq), i32)

    def build(self, items: list[BatchItem]) -> ModelInput:
        B = len(items)
        if B > self.max_seqs:
            raise ValueError(f"batch of {B} sequences exceeds the builder's {self.max_seqs}")
        n_tok = [len(it.tokens) for it in items]
        T = int(sum(n_tok))
        if T > self.max_tokens:
            raise ValueError("batch exceeds max_num_batched_tokens")
        width = max(1, max(len(it.seq.block_table) for it in items))
        if width > self.max_blocks:
            raise ValueError(f"block table of {width} blocks exceeds {self.max_blocks}")
        ids, pos, slot = self.h_ids.numpy(), self.h_pos.numpy(), self.h_slot.numpy()
        smp, qsl, sl, bt = self.h_sample.numpy(), self.h_qsl.numpy(), self.h_sl.numpy(), self.h_bt.numpy()
        qsl[0] = 0
        qsl[1:B + 1] = np.cumsum(n_tok)
        off, ns = 0, 0
        for i, it in enumerate(items):
            n = n_tok[i]
            p = np.arange(it.start, it.start + n, dtype=np.int64)
            table = np.asarray(it.seq.block_table, dtype=np.int64)
            ids[off:off + n] = it.tokens
            pos[off:off + n] = p
            slot[off:off + n] = table[p // BLOCK_SIZE] * BLOCK_SIZE + p % BLOCK_SIZE
            sl[i] = it.start + n
            nb = len(table)
            bt[i, :nb] = table
            bt[i, nb:width] = 0                   # rows are reused across steps: clear stale ids
            if it.sample == "last":
                smp[ns] = off + n - 1
                ns += 1
            elif it.sample == "all":
                smp[ns:ns + n] = np.arange(off, off + n)
                ns += n
            off += n
        nb_ = self.device.type != "cpu"
        self.d_ids[:T].copy_(self.h_ids[:T], non_blocking=nb_)
        self.d_pos[:T].copy_(self.h_pos[:T], non_blocking=nb_)
        self.d_slot[:T].copy_(self.h_slot[:T], non_blocking=nb_)
        self.d_sample[:ns].copy_(self.h_sample[:ns], non_blocking=nb_)
        self.d_qsl[:B + 1].copy_(self.h_qsl[:B + 1], non_blocking=nb_)
        self.d_sl[:B].copy_(self.h_sl[:B], non_blocking=nb_)
        self.d_bt[:B, :width].copy_(self.h_bt[:B, :width], non_blocking=nb_)
        meta = AttentionMetadata(
            query_start_loc=self.d_qsl[:B + 1], seq_lens=self.d_sl[:B],
            block_tables=self.d_bt[:B, :width], slot_mapping=self.d_slot[:T],
            num_decode=num_decode_rows(items), max_query_len=max(n_tok),
            max_seq_len=int(sl[:B].max()))
        return ModelInput(self.d_ids[:T], self.d_pos[:T], meta, self.d_sample[:ns])
