"""A minimal greedy serving loop around the hot path, for end-to-end checks.

Restates the parts of the reference's engine that shape the kernels' inputs: a block allocator
that never hands out the null block 0 (kv/block_allocator.py:16-62), continuous batching with
decodes scheduled first and prompts prefilled in chunks under a token budget
(scheduler/scheduler.py:65-130), an input builder per step (host or device) and graph replay of
pure-decode steps (runner/model_runner.py:20-28). Sampling is greedy argmax.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from turingserve_amd.graphs import DecodeGraphs
from turingserve_amd.metadata import (BatchItem, DeviceInputBuilder, InputBuilder, SeqState,
                                      num_decode_rows)

BLOCK = 16


class BlockAllocator:
    def __init__(self, num_blocks: int) -> None:
        self.free = list(range(num_blocks - 1, 0, -1))     # block 0 is the null block

    def grow(self, seq: SeqState, tokens: int) -> None:
        need = -(-tokens // BLOCK) - len(seq.block_table)
        if need > len(self.free):
            raise RuntimeError("out of KV blocks")
        for _ in range(need):
            seq.block_table.append(self.free.pop())

    def release(self, seq: SeqState) -> None:
        self.free.extend(reversed(seq.block_table))
        seq.block_table = []


@dataclass
class Request:
    prompt: list[int]
    max_tokens: int
    index: int = 0
    seq: SeqState = field(init=False)
    computed: int = 0
    output: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        self.seq = SeqState(list(self.prompt))

    @property
    def done(self) -> bool:
        return len(self.output) >= self.max_tokens


class GreedyEngine:
    def __init__(self, model, num_blocks: int, max_num_batched_tokens: int = 256,
                 max_num_seqs: int = 32, max_model_len: int = 1024, graph_sizes=(),
                 device_metadata: bool = False) -> None:
        self.model = model
        self.kv = model.new_kv_cache(num_blocks)
        self.alloc = BlockAllocator(num_blocks)
        self.budget = max_num_batched_tokens
        self.max_seqs = max_num_seqs
        self.max_blocks = -(-max_model_len // BLOCK)
        self.device_metadata = device_metadata
        make = DeviceInputBuilder if device_metadata else InputBuilder
        self.builder = make(max_num_batched_tokens, max_num_seqs, self.max_blocks, model.device)
        self.graphs = None
        if graph_sizes:
            self.graphs = DecodeGraphs(model, self.kv, graph_sizes, self.max_blocks, max_model_len)
            self.graphs.capture()
        self.graph_steps = 0            # pure-decode steps replayed from a captured graph
        self.mixed_steps = 0            # steps holding decode rows and prompt chunks together
        # (request, output index, argmax, top-2 logit gap, top logit) per sampled token
        self.trace: list[tuple[int, int, int, float, float]] = []

    def _schedule(self, running: list[Request]) -> list[tuple[Request, BatchItem]]:
        """Decodes first (one token each), then prompt chunks while the token budget lasts."""
        plan, budget = [], self.budget
        for r in running:
            if r.computed >= len(r.seq.token_ids) - 1 and r.output and len(plan) < self.max_seqs:
                plan.append((r, 1))
                budget -= 1
        for r in running:
            left = len(r.seq.token_ids) - r.computed
            if r.output or left <= 0 or budget <= 0 or len(plan) >= self.max_seqs:
                continue
            n = min(left, budget)
            plan.append((r, n))
            budget -= n
        items = []
        for r, n in plan:
            self.alloc.grow(r.seq, r.computed + n)
            toks = r.seq.token_ids[r.computed:r.computed + n]
            finishes_prompt = r.computed + n == len(r.seq.token_ids)
            items.append((r, BatchItem(r.seq, r.computed, toks, "last" if finishes_prompt else "none")))
        return items

    @torch.inference_mode()
    def step(self, running: list[Request]) -> None:
        sched = self._schedule(running)
        items = [it for _, it in sched]
        nd = num_decode_rows(items)
        pure_decode = nd == len(items) and all(it.sample == "last" for it in items)
        self.mixed_steps += int(0 < nd < len(items))
        if pure_decode and self.graphs is not None and self.graphs.size_for(len(items)):
            logits = self.graphs.run(items, self.builder if self.device_metadata else None)
            self.graph_steps += 1
        else:
            inp = self.builder.build(items)
            hidden = self.model.forward(inp.input_ids, inp.positions, inp.meta, self.kv)
            logits = self.model.compute_logits(hidden, inp.sample_indices)
        top = logits.topk(2, dim=-1)
        vals, next_ids = top.values.cpu(), top.indices[:, 0].tolist()   # the step waits here
        best, gaps = vals[:, 0].tolist(), (vals[:, 0] - vals[:, 1]).tolist()
        k = 0
        for r, it in sched:
            r.computed += len(it.tokens)
            if it.sample == "last":
                tok = int(next_ids[k])
                self.trace.append((r.index, len(r.output), tok, float(gaps[k]), float(best[k])))
                k += 1
                r.output.append(tok)
                r.seq.token_ids.append(tok)

    def generate(self, prompts: list[list[int]], max_tokens: int) -> list[list[int]]:
        """Greedy outputs of every prompt; `trace` records each sampled argmax with its top-2
        gap and top logit."""
        reqs = [Request(p, max_tokens, i) for i, p in enumerate(prompts)]
        running = list(reqs)
        while running:
            self.step(running)
            for r in [r for r in running if r.done]:
                self.alloc.release(r.seq)
                running.remove(r)
        return [r.output for r in reqs]
