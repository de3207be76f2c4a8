"""One-launch ragged attention (decode splits and prefill tiles side by side) against the oracle
(needs an MI355X).

ts_paged_attention runs the decode rows and the prefill chunks of a batch in one launch (plus
one merge launch) when head_dim is 128, the decode policy is automatic and the workspace is the
size ts_paged_attention_workspace_bytes() asks for; with a workspace sized for the sequential
path it runs the two kernels one after the other. Both must match the oracle
(ops/reference.py:94-111) with the attention criterion of the other kernel tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from turingserve_amd import _native as N
from turingserve_amd import hip_ops as K
from turingserve_amd import synth

from .test_kernels_gpu import DEV, assert_attn, make_paged, meta_of, oracle_attn

pytestmark = pytest.mark.gpu
H, KVH, D = 12, 2, 128


def sizes(meta, B, S):
    cus = N.cu_count(0)
    pf_bound = int(meta.seq_lens[S:].max()) if B > S else 0
    fused = N.lib().ts_paged_attention_workspace_bytes(
        B, S, int(meta.max_query_len), int(meta.max_seq_len), pf_bound, H, KVH, D, 0, 0, cus)
    dec = N.lib().ts_decode_workspace_bytes(0, S, H, KVH, D, int(meta.max_seq_len), 0, cus)
    pf = N.lib().ts_prefill_workspace_bytes(B - S, H, D, int(meta.max_query_len), pf_bound, cus)
    return fused, max(dec, pf), pf_bound


def call(q, kc, vc, meta, ws, nbytes, pf_bound):
    T = q.shape[0]
    out = torch.full((T, H * D), float("nan"), dtype=torch.float16, device=DEV)
    bt, sl, qsl = meta.block_tables, meta.seq_lens, meta.query_start_loc
    N.check(N.lib().ts_paged_attention(
        q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), T, kc.data_ptr(),
        vc.data_ptr(), kc.shape[0], bt.data_ptr(), bt.stride(0), bt.shape[1], sl.data_ptr(),
        qsl.data_ptr(), sl.shape[0], meta.num_decode, int(meta.max_query_len),
        int(meta.max_seq_len), pf_bound, H, KVH, D, D ** -0.5, 0, 0, ws.data_ptr(), nbytes,
        torch.cuda.current_stream().cuda_stream), "paged_attention")
    torch.cuda.synchronize()
    return out


def mixed_case(n_decode, chunks, seed):
    """n_decode decode rows with contexts log-uniform in [256, 4096], then prefill chunks
    (prefix, q_len)."""
    g = torch.Generator().manual_seed(seed)
    ctx = synth.log_uniform_ints(n_decode, 256, 4096, g)
    seq = ctx + [p + n for p, n in chunks]
    ql = [1] * n_decode + [n for _, n in chunks]
    q, kc, vc, qsl, sl, bt = make_paged(seq, H, KVH, D, ql, seed=seed)
    meta = meta_of(qsl, sl, bt, n_decode, ql, q.shape[0])
    ref = oracle_attn(q, kc, vc, qsl, sl, bt, D ** -0.5)
    return [x.to(DEV) for x in (q, kc, vc)], meta, ref


@pytest.mark.parametrize("n_decode,chunks", [
    (48, [(1037, 512)]),                    # the mixed step of config 5
    (1, [(0, 17)]),
    (7, [(100, 128), (0, 300), (2000, 5)]),
    (64, [(63, 129)]),
    (16, [(3000, 1024)]),
])
def test_ragged_fused_and_sequential_match_oracle(n_decode, chunks):
    (q, kc, vc), meta, ref = mixed_case(n_decode, chunks, seed=n_decode)
    B = n_decode + len(chunks)
    fused, seq_need, pf_bound = sizes(meta, B, n_decode)
    # The fused launch needs the decode partials and the prefill partials side by side; when
    # the prefill tiles are not split, the sequential size already suffices for it.
    assert fused >= seq_need
    if n_decode == 48:
        dec = N.lib().ts_decode_workspace_bytes(0, n_decode, H, KVH, D, int(meta.max_seq_len), 0,
                                                N.cu_count(0))
        assert fused > dec, "the config 5 mixed step must split its prefill tiles"
    ws = torch.empty(fused, dtype=torch.uint8, device=DEV)
    assert_attn(call(q, kc, vc, meta, ws, fused, pf_bound), ref, "fused")
    assert_attn(call(q, kc, vc, meta, ws, seq_need, pf_bound), ref, "sequential")
    # through the op namespace (which sizes the workspace for the fused path)
    assert_attn(K.paged_attention(q, kc, vc, meta, D ** -0.5), ref, "paged_attention")


def test_ragged_fused_stale_nan_workspace():
    """Split partials are always written before they are read: a NaN-filled workspace gives
    the same result."""
    (q, kc, vc), meta, ref = mixed_case(48, [(1037, 512)], seed=11)
    fused, _, pf_bound = sizes(meta, 49, 48)
    ws = torch.full((fused // 4 + 64,), float("nan"), dtype=torch.float32, device=DEV)
    assert_attn(call(q, kc, vc, meta, ws.view(torch.uint8), fused, pf_bound), ref, "nan ws")


def test_ragged_padding_decode_rows_are_zero():
    """Decode rows with seq_len 0 (graph padding) are written as zeros in the fused launch."""
    (q, kc, vc), meta, ref = mixed_case(8, [(500, 200)], seed=5)
    meta.seq_lens[2] = 0
    meta.seq_lens[5] = 0
    ref = ref.copy()
    ref[2] = 0.0
    ref[5] = 0.0
    fused, _, pf_bound = sizes(meta, 9, 8)
    ws = torch.empty(fused, dtype=torch.uint8, device=DEV)
    out = call(q, kc, vc, meta, ws, fused, pf_bound)
    assert torch.equal(out[2], torch.zeros_like(out[2])) and torch.equal(out[5], torch.zeros_like(out[5]))
    assert_attn(out, ref, "padding rows")
