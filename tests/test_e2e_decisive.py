"""The end-to-end greedy cases are decisive (CPU): the reference twins' greedy run of every case
keeps a top-2 logit gap of at least MIN_GAP_ULPS fp16 ulps at every sampled step, with chunked
prefill and continuous batching, so the GPU comparison of free-running tokens tests the kernels,
not tie-breaking."""

from __future__ import annotations

import pytest

from tests.e2e_cases import (BUDGET, CASES, MAX_SEQS, MIN_GAP_ULPS, NEW_TOKENS, NUM_BLOCKS,
                             gap_ulps)
from turingserve_amd import get_ops
from turingserve_amd.engine import GreedyEngine
from turingserve_amd.qwen2 import Qwen2Model, random_weights


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_reference_greedy_run_is_decisive(case):
    w = random_weights(case.cfg, "cpu", seed=0, quantization=case.quantization, draw_on="cpu")
    ref = Qwen2Model(case.cfg, w, get_ops("reference"), max_model_len=1024)
    eng = GreedyEngine(ref, NUM_BLOCKS, max_num_batched_tokens=BUDGET, max_num_seqs=MAX_SEQS)
    out = eng.generate(case.prompts(), NEW_TOKENS)
    assert [len(o) for o in out] == [NEW_TOKENS] * len(out)
    margins = gap_ulps(eng.trace)
    assert len(margins) == NEW_TOKENS * len(out)
    assert min(margins) >= MIN_GAP_ULPS, f"smallest top-2 gap {min(margins):.1f} ulps"
    assert eng.mixed_steps > 0          # prefill chunks and decodes shared a step
