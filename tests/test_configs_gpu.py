"""Benchmark configurations 3 and 5 checked at their own workloads (needs an MI355X).

Config 3: the cold 8000-token prefill in four chunks (2048, 2048, 2048, 1856 rows on prefixes 0,
2048, 4096, 6144) at the 1.5B attention shape (12/2 heads, head_dim 128). Each chunk writes its K/V
and runs paged_attention with the split plan the product path chooses; 80 rows per chunk (every
128-row tile boundary and the chunk's ends, plus random rows) are checked against the oracle, and
on every row the split result must agree with the unsplit launch.

Config 5: one mixed step (48 decodes + one 512-token chunk) of a random-init Qwen2 at the 1.5B
dimensions with W8A16 linears, through get_ops("hip") and get_ops("reference") on the same
weights and caches. Every layer is run by both backends on the reference's input to that layer,
and its outputs (MLP output and residual) must agree within LAYER_REL (relative Frobenius norm);
the whole step through each backend must give logits within STEP_REL and the same argmax
wherever the reference's top-2 logit gap exceeds fp16 noise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged as OP
from turingserve_amd import _native as N
from turingserve_amd import hip_ops as K
from turingserve_amd import synth

from .test_kernels_gpu import DEV, assert_attn

pytestmark = pytest.mark.gpu

LAYER_REL = 5e-3          # per-layer relative error bound of the config-5 comparison
STEP_REL = 1e-2           # the whole step's logits (28 layers of differences compound)
LOGIT_NOISE = 0.05


def _rows_to_check(n: int, rng: np.random.Generator) -> np.ndarray:
    edges = {0, 1, n - 2, n - 1}
    for t in range(128, n, 128):
        edges.update((t - 1, t))
    extra = rng.choice(n, size=max(0, 80 - len(edges)), replace=False)
    return np.array(sorted(r for r in edges.union(extra.tolist()) if 0 <= r < n))


@pytest.mark.parametrize("chunk", range(4))
def test_config3_chunk_at_full_size(chunk):
    prefix, n = synth.config3_chunks()[chunk]
    st = synth.config3(chunk, seed=0)
    kc, vc = st.k_cache.to(DEV), st.v_cache.to(DEV)
    qkv = st.qkv.to(DEV)
    q, k, v = st.views(qkv)
    meta = st.meta(DEV)
    K.kv_write(k, v, kc, vc, meta.slot_mapping)
    out = K.paged_attention(q, kc, vc, meta, st.D ** -0.5)
    # the unsplit launch (no workspace) over the same cache
    unsplit = torch.full_like(out, float("nan"))
    bt, sl, qsl = meta.block_tables, meta.seq_lens, meta.query_start_loc
    N.check(N.lib().ts_prefill_attention(
        q.data_ptr(), q.stride(0), q.stride(1), unsplit.data_ptr(), unsplit.stride(0), n,
        kc.data_ptr(), vc.data_ptr(), kc.shape[0], bt.data_ptr(), bt.stride(0), bt.shape[1],
        sl.data_ptr(), qsl.data_ptr(), 1, 0, n, st.H, st.KVH, st.D, st.D ** -0.5,
        torch.cuda.current_stream().cuda_stream), "prefill")
    torch.cuda.synchronize()
    assert_attn(out, unsplit.float().cpu().numpy(), f"chunk {chunk}: split vs unsplit")
    # sampled rows against the oracle, each with its own causal key range
    rows = _rows_to_check(n, np.random.default_rng(chunk))
    qn = q.cpu().numpy()
    kk = OP.gather(kc.cpu().numpy(), bt[0].cpu().numpy(), prefix + n)
    vv = OP.gather(vc.cpu().numpy(), bt[0].cpu().numpy(), prefix + n)
    ref = np.stack([OP.attention_with_mask(qn[r:r + 1], kk[:prefix + r + 1], vv[:prefix + r + 1],
                                           st.D ** -0.5)[0] for r in rows])
    assert_attn(out[torch.from_numpy(rows).to(DEV)], ref,
                f"chunk {chunk} (prefix {prefix}, {n} rows)")


@pytest.fixture(scope="module")
def config5():
    from turingserve_amd import get_ops
    from turingserve_amd.metadata import InputBuilder
    from turingserve_amd.qwen2 import QWEN25_15B, Qwen2Model, random_weights

    cfg = QWEN25_15B
    items, nb, prefix = synth.config5_batch(cfg.vocab_size, seed=0)
    w = random_weights(cfg, DEV, quantization="int8", init_std=0.02, seed=0)
    hip = Qwen2Model(cfg, w, get_ops("hip"), max_model_len=8192)
    ref = Qwen2Model(cfg, w, get_ops("reference"), max_model_len=8192)
    kv = hip.new_kv_cache(nb)
    kv.normal_(0.0, 0.5, generator=torch.Generator(device=DEV).manual_seed(1))
    inp = InputBuilder(1024, 64, 512, DEV).build(items)
    yield hip, ref, kv, inp, prefix
    del hip, ref, kv, w
    torch.cuda.empty_cache()


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float() - b.float()).norm() / b.float().norm())


def test_config5_every_layer_matches_the_reference(config5):
    hip, ref, kv, inp, prefix = config5
    assert inp.input_ids.shape[0] == 560 and inp.meta.num_decode == 48
    kv_h, kv_r = kv.clone(), kv.clone()
    h, res = hip.w.embed_tokens[inp.input_ids], None
    worst = []
    for i in range(len(ref.w.layers)):
        hh, rh = hip.layer_forward(i, h, res, inp.positions, inp.meta, kv_h)
        hr, rr = ref.layer_forward(i, h, res, inp.positions, inp.meta, kv_r)
        e = max(_rel(hh, hr), _rel(rh, rr))
        worst.append(e)
        assert torch.isfinite(hh).all() and e < LAYER_REL, f"layer {i}: relative error {e:.2e}"
        h, res = hr, rr
    print(f"config5 per-layer relative error: max {max(worst):.2e}, mean {np.mean(worst):.2e}")


def test_config5_step_argmax_matches_the_reference(config5):
    hip, ref, kv, inp, prefix = config5
    with torch.inference_mode():
        lh = hip.compute_logits(hip.forward(inp.input_ids, inp.positions, inp.meta, kv.clone()),
                                inp.sample_indices)
        lr = ref.compute_logits(ref.forward(inp.input_ids, inp.positions, inp.meta, kv.clone()),
                                inp.sample_indices)
    assert lh.shape == lr.shape == (49, hip.cfg.vocab_size)
    top = lr.topk(2, dim=-1).values
    decisive = (top[:, 0] - top[:, 1]) > LOGIT_NOISE
    assert int(decisive.sum()) >= 25
    assert torch.equal(lh.argmax(-1)[decisive], lr.argmax(-1)[decisive])
    rel = _rel(lh, lr)
    print(f"config5 step logits relative error {rel:.2e}, {int(decisive.sum())} decisive rows")
    assert rel < STEP_REL
