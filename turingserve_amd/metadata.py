"""Attention metadata of one flat ragged batch, and the builders that produce it.

The kernel input contract is the reference's (runner/attention_metadata.py:10-27,
runner/input_builder.py:41-48): rows [0, num_decode) are decodes with one query token each (q row
index == sequence index), then prefill chunks; ``seq_lens`` is the context length after this
step; ``slot_mapping[t] = table[pos // 16] * 16 + pos % 16`` (-1 = padding row); block-table rows
are padded with block 0, the null block. Two builders produce it: ``InputBuilder`` computes the
arrays on the host in one vectorised pass and uploads them with a single copy, and
``DeviceInputBuilder`` uploads compact per-sequence descriptors and expands them on the GPU
(``ts_step_metadata``).
"""

from __future__ import annotations

import itertools
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


SAMPLE_CODES = {"none": 0, "last": 1, "all": 2}


@dataclass
class StepArrays:
    """The step's metadata as host arrays, before any upload."""

    ids: np.ndarray            # int64 [T]
    positions: np.ndarray      # int64 [T]
    slots: np.ndarray          # int64 [T]
    query_start_loc: np.ndarray  # int32 [B+1]
    seq_lens: np.ndarray       # int32 [B]
    tables: np.ndarray         # int32 [B, width], width >= 1, zero-padded
    sample: np.ndarray         # int64 [S]
    num_decode: int

    def bounds(self) -> dict:
        """The host ints of AttentionMetadata."""
        B, nd = self.seq_lens.shape[0], self.num_decode
        n_tok = np.diff(self.query_start_loc)
        return dict(num_decode=nd, max_query_len=int(n_tok.max(initial=0)),
                    max_seq_len=int(self.seq_lens.max(initial=0)),
                    max_prefill_seq_len=int(self.seq_lens[nd:B].max(initial=0)))


def step_arrays(items: list[BatchItem]) -> StepArrays:
    """Every array of the step from per-item vectors, without a per-token Python loop: a token's
    item comes from repeating item indices by token counts, its position from its offset inside
    the item, its slot from a gather in the padded table. A position whose block lies past the
    item's table raises ValueError (the kernels would have no slot for it). An item with no
    tokens samples nothing."""
    B = len(items)
    if B == 0:
        raise ValueError("a step needs at least one item")
    n_tok = np.fromiter((len(it.tokens) for it in items), np.int64, B)
    start = np.fromiter((it.start for it in items), np.int64, B)
    t_len = np.fromiter((len(it.seq.block_table) for it in items), np.int64, B)
    mode = np.fromiter((SAMPLE_CODES[it.sample] for it in items), np.int64, B)
    ends = np.cumsum(n_tok)
    T = int(ends[-1])
    owner = np.repeat(np.arange(B), n_tok)
    first = ends - n_tok                                   # flat index of each item's token 0
    positions = np.arange(T, dtype=np.int64) - first[owner] + start[owner]
    width = max(1, int(t_len.max()))
    tables = np.zeros((B, width), np.int32)
    tables[np.arange(width)[None, :] < t_len[:, None]] = np.fromiter(
        itertools.chain.from_iterable(it.seq.block_table for it in items), np.int32,
        int(t_len.sum()))
    blk = positions // BLOCK_SIZE
    if T and bool((blk >= t_len[owner]).any()):
        t = int(np.argmax(blk >= t_len[owner]))
        raise ValueError(f"position {int(positions[t])} of item {int(owner[t])} lies past its "
                         f"{int(t_len[owner[t]])}-block table")
    slots = tables[owner, blk].astype(np.int64) * BLOCK_SIZE + positions % BLOCK_SIZE
    flat = np.arange(T)
    sampled = (mode[owner] == 2) | ((mode[owner] == 1) & (flat == ends[owner] - 1))
    leading = (n_tok == 1) & (mode != 2)
    nd = B if bool(leading.all()) else int(np.argmin(leading))
    qsl = np.zeros(B + 1, np.int32)
    qsl[1:] = ends
    return StepArrays(
        ids=np.fromiter(itertools.chain.from_iterable(it.tokens for it in items), np.int64, T),
        positions=positions, slots=slots, query_start_loc=qsl,
        seq_lens=(start + n_tok).astype(np.int32), tables=tables,
        sample=np.flatnonzero(sampled).astype(np.int64), num_decode=nd)


_ALIGN = 256


def _carve(arena: torch.Tensor, sections) -> list[torch.Tensor]:
    """Typed views of a byte arena: one per (dtype, shape) in order, each at a 256-byte aligned
    offset. Returns the views; the arena must be large enough (checked)."""
    views, off = [], 0
    for dtype, shape in sections:
        n = int(np.prod(shape)) if shape else 1
        size = n * torch.empty((), dtype=dtype).element_size()
        if off + size > arena.numel():
            raise ValueError("metadata arena too small")
        views.append(arena[off:off + size].view(dtype).view(*shape))
        off += -(-size // _ALIGN) * _ALIGN
    return views


def _arena_bytes(sections) -> int:
    total = 0
    for dtype, shape in sections:
        n = int(np.prod(shape)) if shape else 1
        total += -(-n * torch.empty((), dtype=dtype).element_size() // _ALIGN) * _ALIGN
    return total


class InputBuilder:
    """Host builder: step_arrays() on the CPU, the arrays packed into one pinned staging arena (on
    a GPU) and sent with ONE host-to-device copy into a device arena whose typed views are the
    step's tensors. The layout is planned per step, so the copy covers only what the step uses.
    The staging arena is rewritten only after the previous step's sampler synchronisation, so no
    copy in flight can still be reading it; the returned tensors are valid until the next build.
    The same ModelInput contract as DeviceInputBuilder (runner/input_builder.py:105-150)."""

    def __init__(self, max_tokens: int, max_seqs: int, max_blocks_per_seq: int, device) -> None:
        self.device = torch.device(device)
        self.max_tokens, self.max_seqs, self.max_blocks = max_tokens, max_seqs, max_blocks_per_seq
        cap = _arena_bytes(self._sections(max_tokens, max_tokens, max_seqs, max_blocks_per_seq))
        on_gpu = self.device.type == "cuda"
        self._stage = torch.zeros(cap, dtype=torch.uint8, pin_memory=on_gpu)
        self._arena = torch.zeros(cap, dtype=torch.uint8, device=self.device)

    @staticmethod
    def _sections(T: int, S: int, B: int, width: int):
        i64, i32 = torch.int64, torch.int32
        return [(i64, (T,)), (i64, (T,)), (i64, (T,)), (i64, (S,)), (i32, (B + 1,)), (i32, (B,)),
                (i32, (B, width))]

    def build(self, items: list[BatchItem]) -> ModelInput:
        B = len(items)
        if B > self.max_seqs:
            raise ValueError(f"batch of {B} sequences exceeds the builder's {self.max_seqs}")
        if sum(len(it.tokens) for it in items) > self.max_tokens:
            raise ValueError("batch exceeds max_num_batched_tokens")
        a = step_arrays(items)
        width = a.tables.shape[1]
        if width > self.max_blocks:
            raise ValueError(f"block table of {width} blocks exceeds {self.max_blocks}")
        T, S = a.ids.shape[0], a.sample.shape[0]
        sections = self._sections(T, S, B, width)
        used = _arena_bytes(sections)
        host = _carve(self._stage, sections)
        for view, arr in zip(host, (a.ids, a.positions, a.slots, a.sample, a.query_start_loc,
                                    a.seq_lens, a.tables)):
            view.numpy()[...] = arr
        self._arena[:used].copy_(self._stage[:used], non_blocking=self.device.type == "cuda")
        ids, pos, slots, sample, qsl, sl, bt = _carve(self._arena, sections)
        meta = AttentionMetadata(query_start_loc=qsl, seq_lens=sl, block_tables=bt,
                                 slot_mapping=slots, **a.bounds())
        return ModelInput(ids, pos, meta, sample)


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
    """Builds the step's metadata on the GPU (ts_step_metadata) from one packed upload of
    per-sequence descriptors instead of the per-token host arrays of InputBuilder; the same
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
