"""Kernel variants on the GPU: every W8A16 variant and split count against the float64 oracle
(oracle/quant.py), and a tuning run whose table the ops then follow (the reference's tuner
measures per-bucket configs the same way, autopilot/tuner.py:116-134)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant as OQ
from turingserve_amd import hip_ops as K
from turingserve_amd import reference_ops as R
from turingserve_amd import tuner as T

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _restore_active():
    saved = T.ACTIVE
    yield
    T.set_active(saved)


def _problem(M, N, Kd, seed, fp16_scale=False):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, Kd, generator=g) * 0.05
    wq, sc = OQ.quantize(w.numpy())
    x = torch.randn(M, Kd, generator=g).half()
    bias = (torch.randn(N, generator=g) * 0.1).half()
    scale = torch.from_numpy(sc)
    ref = OQ.w8a16(x.numpy(), wq, sc, bias.numpy(), np.float64)
    if fp16_scale:
        scale = scale.half()
        ref = OQ.w8a16(x.numpy(), wq, scale.float().numpy(), bias.numpy(), np.float64)
    return (x.to(DEV), torch.from_numpy(wq).to(DEV), scale.to(DEV), bias.to(DEV)), ref


@pytest.mark.parametrize("M,N,Kd", [(1, 2048, 1536), (20, 1000, 520), (64, 1536, 8960),
                                    (300, 2048, 1536), (129, 260, 1032),
                                    (1, 1536, 8960), (3, 260, 1040),    # VALU path, ragged N
                                    (2, 1000, 520)])                    # K % 16 != 0: skinny
def test_every_variant_matches_the_oracle(M, N, Kd):
    (x, wq, sc, b), ref = _problem(M, N, Kd, seed=M + N, fp16_scale=M % 2 == 0)
    auto = K.w8a16_linear(x, wq, sc, b)
    assert torch.equal(auto, K.w8a16_linear(x, wq, sc, b, cfg=(0, 0)))
    for v, s in T.w8a16_candidates(M) + [(3, 3), (2, 7)]:
        y = K.w8a16_linear(x, wq, sc, b, cfg=(v, s)).float().cpu().numpy()
        assert np.isfinite(y).all(), (v, s)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-3, (v, s)


def test_tuned_w8a16_table_is_followed():
    shapes, ms = [(2048, 1536), (1536, 8960)], [16, 768]         # bucket values
    table = T.tune_w8a16(torch, shapes, ms, DEV)
    for (N, Kd) in shapes:
        for M in ms:
            c = table.records("w8a16")[(N, Kd, M)]
            assert (c["variant"], c["splits"]) in T.w8a16_candidates(M) and c["us"] > 0
    T.set_active(table)
    (x, wq, sc, b), _ = _problem(560, 1536, 8960, seed=1)
    c = table.records("w8a16")[(1536, 8960, 768)]                 # M = 560 rounds up to 768
    assert T.w8a16_choice(1536, 8960, 560) == (c["variant"], c["splits"])
    assert torch.equal(K.w8a16_linear(x, wq, sc, b),
                       K.w8a16_linear(x, wq, sc, b, cfg=(c["variant"], c["splits"])))


def test_tuned_decode_table_is_followed():
    from turingserve_amd.metadata import AttentionMetadata

    H, KVH, D = 12, 2, 128
    table = T.tune_decode(torch, H, KVH, D, [4], [256, 2048], DEV)
    T.set_active(table)
    g = torch.Generator(device=DEV).manual_seed(0)
    kc = torch.randn(600, KVH, 16, D, generator=g, device=DEV).half()
    vc = torch.randn(600, KVH, 16, D, generator=g, device=DEV).half()
    S, L = 4, 1500
    bt = torch.randperm(599, generator=g, device=DEV)[:S * 94].add(1).view(S, 94).int()
    meta = AttentionMetadata(torch.arange(S + 1, device=DEV, dtype=torch.int32),
                             torch.tensor([L, 700, 1, 1333], device=DEV, dtype=torch.int32), bt,
                             torch.zeros(S, device=DEV, dtype=torch.int64), S, 1, L)
    q = torch.randn(S, H, D, generator=g, device=DEV).half()
    ver, part = T.decode_choice(S, L)
    assert ver in ("v2", "v3")
    got = K.paged_attention(q, kc, vc, meta, D ** -0.5)
    assert torch.equal(got, K.paged_attention(q, kc, vc, meta, D ** -0.5, decode_version=ver,
                                              partition=part))
    want = R.paged_attention(q, kc, vc, meta, D ** -0.5)
    assert (got.float() - want.float()).abs().max() < 1e-2


def test_tuned_decode_choice_is_for_pure_decode_batches_only():
    """A tuned fixed decode partition applies to pure-decode batches; a mixed batch keeps the
    library's own-length plan, the one that runs its decode rows and prefill tiles in one
    launch, so its output equals the untuned call's bit for bit."""
    from .test_kernels_gpu import make_paged, meta_of

    H, KVH, D = 12, 2, 128
    seq, ql = [900, 40, 1700, 300 + 256], [1, 1, 1, 256]
    q, kc, vc, qsl, sl, bt = make_paged(seq, H, KVH, D, ql, seed=5)
    meta = meta_of(qsl, sl, bt, 3, ql, q.shape[0])
    q, kc, vc = q.to(DEV), kc.to(DEV), vc.to(DEV)
    T.set_active(T.VariantTable())
    untuned = K.paged_attention(q, kc, vc, meta, D ** -0.5)
    table = T.VariantTable()
    table.set("decode", (3, 2048), {"version": "v3", "partition": 256, "us": 1.0})
    T.set_active(table)
    assert T.decode_choice(3, int(meta.max_seq_len)) == ("v3", 256)
    assert torch.equal(K.paged_attention(q, kc, vc, meta, D ** -0.5), untuned)
    # the same decode rows alone follow the table
    dmeta = meta_of(qsl[:4], sl[:3], bt[:3], 3, [1, 1, 1], 3)
    assert torch.equal(K.paged_attention(q[:3], kc, vc, dmeta, D ** -0.5),
                       K.paged_attention(q[:3], kc, vc, dmeta, D ** -0.5, decode_version="v3",
                                         partition=256))
