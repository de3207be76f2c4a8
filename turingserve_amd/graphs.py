"""hipGraph capture and replay of pure-decode steps (runner/cuda_graphs.py:15-78).

A graph per batch size B is captured over static input buffers; replay copies the n real decode
rows in and pads up to the captured size with padding rows (slot -1 so kv_write skips them,
seq_len 0 so attention writes zeros, token/position 0, zeroed block tables). Inside a graph
max_seq_len = max_model_len, which fixes the split-K grid of the decode kernel. Nothing captured
allocates outside the graph pool or synchronises with the host; the decode kernels run with the
library's workspace from the same pool. Graphs are captured after an eager warm-up of every
size, largest first, sharing one memory pool.
"""

from __future__ import annotations

import torch

from turingserve_amd.metadata import AttentionMetadata, ModelInput


class HipGraphRunner:
    def __init__(self, model, kv_cache: torch.Tensor, sizes: tuple[int, ...],
                 max_blocks_per_seq: int, max_model_len: int, device) -> None:
        self.model, self.kv_cache, self.device = model, kv_cache, device
        self.sizes = sorted(set(sizes))
        self.max_b = self.sizes[-1]
        self.max_model_len = max_model_len
        V = model.cfg.vocab_size
        i32, i64 = torch.int32, torch.int64
        self.ids = torch.zeros(self.max_b, dtype=i64, device=device)
        self.pos = torch.zeros(self.max_b, dtype=i64, device=device)
        self.slot = torch.full((self.max_b,), -1, dtype=i64, device=device)
        self.seq_lens = torch.zeros(self.max_b, dtype=i32, device=device)
        self.bt = torch.zeros(self.max_b, max_blocks_per_seq, dtype=i32, device=device)
        self.qsl = torch.arange(self.max_b + 1, dtype=i32, device=device)
        self.sample_idx = torch.arange(self.max_b, dtype=i64, device=device)
        self.logits = torch.zeros(self.max_b, V, dtype=torch.float32, device=device)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}

    def _meta(self, B: int) -> AttentionMetadata:
        return AttentionMetadata(
            query_start_loc=self.qsl[:B + 1], seq_lens=self.seq_lens[:B], block_tables=self.bt[:B],
            slot_mapping=self.slot[:B], num_decode=B, max_query_len=1,
            max_seq_len=self.max_model_len, in_graph=True)

    def _forward(self, B: int) -> None:
        hidden = self.model.forward(self.ids[:B], self.pos[:B], self._meta(B), self.kv_cache)
        self.logits[:B] = self.model.compute_logits(hidden, self.sample_idx[:B])

    def capture(self) -> None:
        for B in self.sizes:                  # eager warm-up of every size
            for _ in range(2):
                self._forward(B)
        torch.cuda.synchronize()
        pool = torch.cuda.graph_pool_handle()
        for B in reversed(self.sizes):        # largest first so smaller graphs share the pool
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self._forward(B)
            self.graphs[B] = g
        torch.cuda.synchronize()

    def can_replay(self, n: int) -> bool:
        return 0 < n <= self.max_b and bool(self.graphs)

    def replay(self, inp: ModelInput, n: int) -> torch.Tensor:
        """Copy the n real decode rows into the static buffers, pad to the graph size, replay;
        returns the logits rows [n, V] (valid until the next replay)."""
        B = next(s for s in self.sizes if s >= n)
        self.ids[:n].copy_(inp.input_ids[:n])
        self.pos[:n].copy_(inp.positions[:n])
        self.slot[:n].copy_(inp.meta.slot_mapping[:n])
        self.seq_lens[:n].copy_(inp.meta.seq_lens[:n])
        self.bt[:B].zero_()
        w = inp.meta.block_tables.shape[1]
        self.bt[:n, :w].copy_(inp.meta.block_tables[:n])
        if B > n:
            self.ids[n:B].zero_()
            self.pos[n:B].zero_()
            self.slot[n:B].fill_(-1)
            self.seq_lens[n:B].zero_()
        self.graphs[B].replay()
        return self.logits[:n]

    def replay_items(self, items, builder) -> torch.Tensor:
        """The same with the step's metadata built on the device (DeviceInputBuilder.build_into):
        the decode rows and the padding go straight into the static buffers, one upload and one
        launch instead of the copies and fills above."""
        n = len(items)
        B = next(s for s in self.sizes if s >= n)
        builder.build_into(items, B, self.ids, self.pos, self.slot, self.qsl, self.seq_lens,
                           self.bt)
        self.graphs[B].replay()
        return self.logits[:n]
