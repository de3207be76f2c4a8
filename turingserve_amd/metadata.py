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
    # Host bound of the prefill rows' seq_lens (0: unknown, max_seq_len applies). Not a field of
    # the reference's metadata: it only sizes the prefill kernel's split plan.
    max_prefill_seq_len: int = 0


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
        max_seq_len=max(seq_lens),
        max_prefill_seq_len=max(seq_lens[num_decode_rows(items):], default=0))
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
            max_seq_len=int(sl[:B].max()),
            max_prefill_seq_len=int(sl[num_decode_rows(items):B].max(initial=0)))
        return ModelInput(self.d_ids[:T], self.d_pos[:T], meta, self.d_sample[:ns])


SAMPLE_CODES = {"none": 0, "last": 1, "all": 2}
DESC_WORDS = 5


def pack_step(items: list[BatchItem], out: np.ndarray | None = None) -> tuple[np.ndarray, int, int, int]:
    """The compact int32 upload that ts_step_metadata expands on the device: per item the
    descriptor {start, n_tokens, sample code, table offset, table length}, then every token id,
    then every block table, concatenated. Written into `out` (e.g. a pinned buffer's view) when
    given. Returns (packed words, num_tokens, num_block_ids, num_samples); an item with no tokens
    samples nothing."""
    B = len(items)
    n_tok = np.fromiter((len(it.tokens) for it in items), np.int64, B)
    t_len = np.fromiter((len(it.seq.block_table) for it in items), np.int64, B)
    T, NB = int(n_tok.sum()), int(t_len.sum())
    total = DESC_WORDS * B + T + NB
    buf = np.empty(total, np.int32) if out is None else out[:total]
    desc = buf[:DESC_WORDS * B].reshape(B, DESC_WORDS)
    desc[:, 0] = np.fromiter((it.start for it in items), np.int64, B)
    desc[:, 1] = n_tok
    codes = np.fromiter((SAMPLE_CODES[it.sample] for it in items), np.int64, B)
    desc[:, 2] = codes
    desc[:, 3] = np.cumsum(t_len) - t_len
    desc[:, 4] = t_len
    o = DESC_WORDS * B
    for it in items:
        n = len(it.tokens)
        buf[o:o + n] = it.tokens
        o += n
    for it in items:
        n = len(it.seq.block_table)
        buf[o:o + n] = it.seq.block_table
        o += n
    S = int(((codes == 1) & (n_tok > 0)).sum() + n_tok[codes == 2].sum())
    return buf, T, NB, S


class DeviceInputBuilder:
    """Builds the step's metadata on the GPU (ts_step_metadata) from one packed upload instead of
    the host arrays and seven copies of InputBuilder (runner/input_builder.py:81-150); the same
    ModelInput contract. The pinned upload buffer is rewritten only after the previous step's
    sampler synchronisation, as with InputBuilder. build_into() writes a pure-decode batch
    straight into a captured graph's static buffers, padded to the graph size
    (runner/cuda_graphs.py:62-78)."""

    def __init__(self, max_tokens: int, max_seqs: int, max_blocks_per_seq: int, device) -> None:
        from turingserve_amd import _native

        self._native = _native
        _native.lib()                               # fail now, loudly, if the library is missing
        self.device = torch.device(device)
        i32, i64 = torch.int32, torch.int64
        self.max_tokens, self.max_seqs, self.max_blocks = max_tokens, max_seqs, max_blocks_per_seq
        cap = DESC_WORDS * max_seqs + max_tokens + max_seqs * max_blocks_per_seq
        self.h_packed = torch.zeros(cap, dtype=i32, pin_memory=True)
        self.d_packed = torch.zeros(cap, dtype=i32, device=self.device)
        dev = lambda *shape, dtype: torch.zeros(*shape, dtype=dtype, device=self.device)
        self.d_ids, self.d_pos = dev(max_tokens, dtype=i64), dev(max_tokens, dtype=i64)
        self.d_slot, self.d_sample = dev(max_tokens, dtype=i64), dev(max_tokens, dtype=i64)
        self.d_qsl, self.d_sl = dev(max_seqs + 1, dtype=i32), dev(max_seqs, dtype=i32)
        self.d_bt = dev(max_seqs, max_blocks_per_seq, dtype=i32)

    def _upload(self, items: list[BatchItem]) -> tuple[int, int, int, int]:
        B = len(items)
        if B > self.max_seqs:
            raise ValueError(f"batch of {B} sequences exceeds the builder's {self.max_seqs}")
        width = max(1, max((len(it.seq.block_table) for it in items), default=1))
        if width > self.max_blocks:
            raise ValueError(f"block table of {width} blocks exceeds {self.max_blocks}")
        if sum(len(it.tokens) for it in items) > self.max_tokens:
            raise ValueError("batch exceeds max_num_batched_tokens")
        words, T, NB, S = pack_step(items, self.h_packed.numpy())
        n = words.size
        self.d_packed[:n].copy_(self.h_packed[:n], non_blocking=True)
        return T, NB, S, width

    def _launch(self, B, pad, T, NB, width, ids, pos, slot, qsl, sl, bt, sample) -> None:
        N = self._native
        stream = torch.cuda.current_stream(self.device).cuda_stream
        ptr = lambda t: None if t is None else t.data_ptr()
        N.check(N.lib().ts_step_metadata(ptr(self.d_packed), B, T, NB, pad, width, bt.stride(0),
                                         ptr(ids), ptr(pos), ptr(slot), ptr(qsl), ptr(sl),
                                         ptr(bt), ptr(sample), stream), "step_metadata")

    def build(self, items: list[BatchItem]) -> ModelInput:
        B = len(items)
        T, NB, S, width = self._upload(items)
        self._launch(B, B, T, NB, width, self.d_ids, self.d_pos, self.d_slot, self.d_qsl,
                     self.d_sl, self.d_bt, self.d_sample)
        n_tok = [len(it.tokens) for it in items]
        meta = AttentionMetadata(
            query_start_loc=self.d_qsl[:B + 1], seq_lens=self.d_sl[:B],
            block_tables=self.d_bt[:B, :width], slot_mapping=self.d_slot[:T],
            num_decode=num_decode_rows(items), max_query_len=max(n_tok),
            max_seq_len=max(it.start + n for it, n in zip(items, n_tok)),
            max_prefill_seq_len=max((it.start + n for it, n in
                                     list(zip(items, n_tok))[num_decode_rows(items):]), default=0))
        return ModelInput(self.d_ids[:T], self.d_pos[:T], meta, self.d_sample[:S])

    def build_into(self, items: list[BatchItem], pad_to: int, ids: torch.Tensor,
                   pos: torch.Tensor, slot: torch.Tensor, qsl: torch.Tensor, seq_lens: torch.Tensor,
                   block_tables: torch.Tensor) -> None:
        """Pure-decode items (one token each) into static buffers of a graph captured for pad_to
        rows: rows len(items) .. pad_to - 1 become padding rows; the table rows are written over
        the buffers' full width."""
        B = len(items)
        if any(len(it.tokens) != 1 for it in items) or not B <= pad_to <= ids.numel():
            raise ValueError("build_into: one token per item and len(items) <= pad_to <= buffer rows")
        T, NB, S, _ = self._upload(items)
        self._launch(B, pad_to, T, NB, block_tables.shape[1], ids, pos, slot, qsl, seq_lens,
                     block_tables, None)
