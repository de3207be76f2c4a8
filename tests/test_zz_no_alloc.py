"""ts_decode_attention_kv_write_noalloc (needs an MI355X): the fused kv_write + decode attention
with its split-K scratch in the library's static device array instead of a workspace argument.
Called through the C ABI, it must leave the same caches and outputs, bit for bit, as
ts_decode_attention_kv_write with a workspace (the same kernels and plan), on two calls in a row
(the second with a smaller batch, over the first call's leftover scratch), and it must reject a
batch whose split scratch exceeds TS_NOALLOC_SCRATCH_BYTES before launching anything."""

from __future__ import annotations

import pytest
import torch

from turingserve_amd import _native as N
from turingserve_amd import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, KVH, D = 12, 2, 128


def _batch(num_seqs, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    ctx = synth.log_uniform_ints(num_seqs, lo, hi, g)
    st = synth.make_step(H, KVH, D, sum(-(-c // 16) for c in ctx) + 8,
                         [(c - 1, 1) for c in ctx], gen=g)
    return st


def _call(st, noalloc, version=0, partition=0, max_seq_len=None):
    kc, vc = st.k_cache.to(DEV), st.v_cache.to(DEV)
    qkv = st.qkv.to(DEV)
    q, k, v = st.views(qkv)
    m = st.meta(DEV)
    S = st.T
    out = torch.full((S, H * D), float("nan"), dtype=torch.float16, device=DEV)
    bt, sl, slots = m.block_tables, m.seq_lens, m.slot_mapping
    stream = torch.cuda.current_stream().cuda_stream
    head = (version, q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
            k.stride(0), k.stride(1), v.stride(0), v.stride(1), slots.data_ptr(),
            out.data_ptr(), out.stride(0), kc.data_ptr(), vc.data_ptr(), kc.shape[0],
            bt.data_ptr(), bt.stride(0), bt.shape[1], sl.data_ptr(), S, H, KVH, D, D ** -0.5,
            int(m.max_seq_len if max_seq_len is None else max_seq_len), partition)
    lib = N.lib()
    if noalloc:
        status = lib.ts_decode_attention_kv_write_noalloc(*head, stream)
    else:
        nb = lib.ts_decode_workspace_bytes(version, S, H, KVH, D, int(m.max_seq_len), partition,
                                           N.cu_count(0))
        ws = torch.full((max(nb, 256) // 4,), float("nan"), dtype=torch.float32, device=DEV)
        status = lib.ts_decode_attention_kv_write(*head, ws.data_ptr(), nb, stream, None, 0)
    torch.cuda.synchronize()
    return status, out, kc, vc


@pytest.mark.parametrize("version,partition", [(0, 0), (3, 512)])
def test_noalloc_equals_workspace_entry_on_two_calls(version, partition):
    for st in (_batch(64, 128, 4096, seed=0), _batch(17, 16, 1500, seed=1)):
        ref = _call(st, False, version, partition)
        got = _call(st, True, version, partition)
        assert ref[0] == N.TS_OK and got[0] == N.TS_OK, N.last_error()
        assert N.last_error() == ""
        for a, b in zip(ref[1:], got[1:]):
            assert torch.equal(a, b)


def test_noalloc_rejects_a_batch_beyond_its_scratch():
    # a host bound of 32768 tokens: the own-length plan reserves 32 split rows per sequence,
    # 192 x 32 rows of 12 heads, more than the scratch holds
    st = _batch(192, 64, 256, seed=2)
    need = N.lib().ts_decode_workspace_bytes(3, st.T, H, KVH, D, 32768, 0, N.cu_count(0))
    assert need > N.TS_NOALLOC_SCRATCH_BYTES
    status, out, kc, vc = _call(st, True, version=3, max_seq_len=32768)
    assert status == N.TS_ERR_WORKSPACE
    assert "static scratch" in N.last_error()
    assert torch.isnan(out).all()                              # nothing was launched
    assert torch.equal(kc.cpu(), st.k_cache)
