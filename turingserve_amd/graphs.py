"""hipGraph replay of pure-decode steps (the role of runner/cuda_graphs.py:15-78).

One static decode batch lives in a single device byte arena: typed views for the token ids,
positions, slots, seq_lens, block tables (the rows a step changes, laid out first and contiguous)
and for query_start_loc and the sample rows (written once: every decode row is its own sequence
and samples itself). A graph is captured per batch size of the ladder, each over the first B rows
of those views. A step refills the changing rows in one go, either from the host (numpy into a
pinned mirror of the arena, then one host-to-device copy) or on the device
(``DeviceInputBuilder.build_into``, one upload and one launch), then replays the smallest graph
that holds it. Rows past the step's sequences are padding: slot -1 (kv_write skips it), seq_len 0
(attention writes zeros), token and position 0, an all-zero table row.

Inside a graph the decode kernels take the own-length split schedule with max_seq_len =
max_model_len (its plan depends on the batch size and that bound, not on the lengths), so one
graph serves every context length up to the table width. Nothing captured synchronises with the host or allocates outside the graphs' shared pool.
"""

from __future__ import annotations

import numpy as np
import torch

from turingserve_amd.metadata import AttentionMetadata, BatchItem, _arena_bytes, _carve


class StaticDecodeBatch:
    """The captured graphs' inputs: views of one device arena (and its pinned host mirror)."""

    def __init__(self, rows: int, width: int, device) -> None:
        self.rows, self.width = rows, width
        i64, i32 = torch.int64, torch.int32
        self._sections = [(i64, (rows,)), (i64, (rows,)), (i64, (rows,)), (i32, (rows,)),
                          (i32, (rows, width)), (i32, (rows + 1,)), (i64, (rows,))]
        size = _arena_bytes(self._sections)
        self._dirty = _arena_bytes(self._sections[:5])          # ids .. tables
        self.arena = torch.zeros(size, dtype=torch.uint8, device=device)
        self.stage = torch.zeros(size, dtype=torch.uint8, pin_memory=True)
        (self.ids, self.pos, self.slots, self.seq_lens, self.tables, self.qsl,
         self.sample) = _carve(self.arena, self._sections)
        host = _carve(self.stage, self._sections)
        self._h = [t.numpy() for t in host]
        self._h[2][:] = -1                                      # every row starts as padding
        self._h[5][:] = np.arange(rows + 1)
        self._h[6][:] = np.arange(rows)
        self.arena.copy_(self.stage)
        self._copied: torch.cuda.Event | None = None    # the last stage -> arena copy

    def meta(self, B: int, max_model_len: int) -> AttentionMetadata:
        return AttentionMetadata(
            query_start_loc=self.qsl[:B + 1], seq_lens=self.seq_lens[:B],
            block_tables=self.tables[:B], slot_mapping=self.slots[:B], num_decode=B,
            max_query_len=1, max_seq_len=max_model_len, in_graph=True)

    def fill_from_host(self, items: list[BatchItem], B: int) -> None:
        """Rows 0 .. len(items)-1 from the items (one token each), rows up to B padding; one
        copy of the changing part of the arena. The copy reads the pinned stage asynchronously:
        before the stage is written again, the previous call's copy is waited for (an event
        recorded after it), so two calls in a row without a synchronisation cannot race."""
        if self._copied is not None:
            self._copied.synchronize()
        n = len(items)
        ids, pos, slots, sl, tables = self._h[:5]
        start = np.fromiter((it.start for it in items), np.int64, n)
        t_len = np.fromiter((len(it.seq.block_table) for it in items), np.int64, n)
        if n and int(t_len.max()) > self.width:
            raise ValueError(f"block table of {int(t_len.max())} blocks exceeds {self.width}")
        if n and bool((start // 16 >= t_len).any()):
            raise ValueError("a decode position lies past its block table")
        ids[:n] = np.fromiter((it.tokens[0] for it in items), np.int64, n)
        pos[:n] = start
        sl[:n] = start + 1
        tables[:B] = 0
        for r, it in enumerate(items):
            tables[r, :len(it.seq.block_table)] = it.seq.block_table
        slots[:n] = tables[np.arange(n), start // 16].astype(np.int64) * 16 + start % 16
        ids[n:B], pos[n:B], slots[n:B], sl[n:B] = 0, 0, -1, 0
        self.arena[:self._dirty].copy_(self.stage[:self._dirty], non_blocking=True)
        if self._copied is None:
            self._copied = torch.cuda.Event()
        self._copied.record()


class DecodeGraphs:
    """Pure-decode steps captured once per batch size of `sizes` and replayed with the step's rows
    written into the static batch."""

    def __init__(self, model, kv_cache: torch.Tensor, sizes, max_blocks_per_seq: int,
                 max_model_len: int) -> None:
        self.model, self.kv_cache = model, kv_cache
        self.ladder = sorted(set(int(s) for s in sizes))
        if not self.ladder or self.ladder[0] < 1:
            raise ValueError("graph sizes must be positive")
        self.max_model_len = max_model_len
        self.batch = StaticDecodeBatch(self.ladder[-1], max_blocks_per_seq, kv_cache.device)
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._logits: dict[int, torch.Tensor] = {}

    def _step(self, B: int) -> torch.Tensor:
        b = self.batch
        hidden = self.model.forward(b.ids[:B], b.pos[:B], b.meta(B, self.max_model_len),
                                    self.kv_cache)
        return self.model.compute_logits(hidden, b.sample[:B])

    def capture(self) -> None:
        """One eager run per size (the padding rows write nothing), then the captures. The graphs
        share one memory pool; each graph's logits stay allocated, so no later capture reuses
        them. Capturing the largest first lets the smaller graphs fit in what it reserved."""
        with torch.inference_mode():
            for B in self.ladder:
                self._step(B)
            torch.cuda.synchronize()
            pool = torch.cuda.graph_pool_handle()
            for B in sorted(self.ladder, reverse=True):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=pool):
                    self._logits[B] = self._step(B)
                self._graphs[B] = g
        torch.cuda.synchronize()

    def size_for(self, n: int) -> int | None:
        """The smallest captured size that holds n decode rows (None if none does)."""
        for B in self.ladder:
            if B >= n and B in self._graphs:
                return B
        return None

    def run(self, items: list[BatchItem], device_builder=None) -> torch.Tensor:
        """Replay the step of `items` (pure decode, one token each); logits [len(items), V] fp32,
        valid until the next replay of the same size. With `device_builder` (a
        DeviceInputBuilder) the rows are written on the GPU, else from the host."""
        n = len(items)
        B = self.size_for(n)
        if B is None or any(len(it.tokens) != 1 for it in items):
            raise ValueError(f"no captured decode graph for {n} single-token rows")
        b = self.batch
        if device_builder is not None:
            device_builder.build_into(items, B, b.ids, b.pos, b.slots, b.qsl, b.seq_lens, b.tables)
        else:
            b.fill_from_host(items, B)
        self._graphs[B].replay()
        return self._logits[B][:n]
