"""Pinning the oracle (CPU). The reference stores no golden vectors for this path, so every oracle
function is checked against something independent of its own formula: a pure-Python fp64 brute
force, closed forms and special cases, invariants (paged == contiguous, split-K == single pass,
scatter == explicit loop) and the quantisation error bound. Each check is chosen so that a
plausible slip (mask off by one, wrong GQA head map, wrong merge weight, transposed weight) fails.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import paged as OP
from oracle import quant as OQ


def rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float16)


# ------------------------------------------------------------------------------------------
# attention_with_mask vs pure-Python loops
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("Tq,Tk,H,KVH,D", [(1, 1, 2, 1, 4), (1, 9, 4, 2, 8), (5, 5, 3, 3, 4),
                                           (4, 11, 6, 2, 8), (7, 20, 7, 1, 16), (3, 3, 4, 2, 16)])
def test_attention_matches_brute_force(Tq, Tk, H, KVH, D):
    q, k, v = rnd((Tq, H, D), 1), rnd((Tk, KVH, D), 2), rnd((Tk, KVH, D), 3)
    got = OP.attention_with_mask(q, k, v, D ** -0.5, np.float64)
    want = OP.attention_brute(q, k, v, D ** -0.5)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    got32 = OP.attention_with_mask(q, k, v, D ** -0.5, np.float32)
    np.testing.assert_allclose(got32, want, rtol=1e-5, atol=1e-5)


def test_attention_special_cases():
    D = 8
    k, v = rnd((6, 1, D), 4), rnd((6, 1, D), 5)
    # one visible key: the output is that value row exactly
    q = rnd((6, 1, D), 6)
    out = OP.attention_with_mask(q, k, v, 0.3, np.float64)
    np.testing.assert_array_equal(out[0], v[0, 0].astype(np.float64))
    # zero query: uniform weights over the visible prefix (row i sees keys 0..i)
    out = OP.attention_with_mask(np.zeros((6, 1, D), np.float16), k, v, 1.0, np.float64)
    for i in range(6):
        np.testing.assert_allclose(out[i], v[: i + 1, 0].astype(np.float64).mean(0), rtol=1e-12)
    # bottom-right alignment: 2 queries over 5 keys, the first sees keys 0..3
    out = OP.attention_with_mask(np.zeros((2, 1, D), np.float16), k[:5], v[:5], 1.0, np.float64)
    np.testing.assert_allclose(out[0], v[:4, 0].astype(np.float64).mean(0), rtol=1e-12)


def test_gqa_head_map_is_h_div_g():
    """Query head h reads KV head h // G (repeat_interleave): distinct constant V per KV head."""
    H, KVH, D = 6, 3, 4
    k = np.zeros((5, KVH, D), np.float16)
    v = np.zeros((5, KVH, D), np.float16)
    for j in range(KVH):
        v[:, j, :] = j + 1
    out = OP.attention_with_mask(rnd((1, H, D), 7), k, v, 1.0, np.float64).reshape(H, D)
    for h in range(H):
        np.testing.assert_allclose(out[h], h // (H // KVH) + 1, rtol=1e-12)


# ------------------------------------------------------------------------------------------
# slot mapping, kv_write, gather, paged == contiguous
# ------------------------------------------------------------------------------------------
def test_slot_mapping_closed_form():
    table = [7, 3, 11, 2]
    pos = list(range(64))
    got = OP.slot_mapping(table, pos)
    assert got.tolist() == [table[p // 16] * 16 + p % 16 for p in pos]


def test_kv_write_equals_explicit_loop():
    NB, KVH, D, T = 8, 2, 4, 20
    k, v = rnd((T, KVH, D), 8), rnd((T, KVH, D), 9)
    slots = np.random.default_rng(0).permutation(NB * 16)[:T].astype(np.int64)
    slots[::4] = -1
    kc, vc = rnd((NB, KVH, 16, D), 10), rnd((NB, KVH, 16, D), 11)
    kl, vl = kc.copy(), vc.copy()
    for t in range(T):
        s = slots[t]
        if s < 0:
            continue
        for h in range(KVH):
            kl[s // 16, h, s % 16] = k[t, h]
            vl[s // 16, h, s % 16] = v[t, h]
    OP.kv_write(k, v, kc, vc, slots)
    assert np.array_equal(kc, kl) and np.array_equal(vc, vl)


@pytest.mark.parametrize("lens", [[5, 16, 17, 100], [1], [333, 2, 64]])
def test_paged_equals_contiguous(lens):
    """Scatter contiguous K/V through shuffled block tables, gather them back through paged
    attention: identical results (tests/correctness/test_paged_engine.py:46-63 idea)."""
    H, KVH, D = 4, 2, 8
    rng = np.random.default_rng(sum(lens))
    nbs = [-(-L // 16) for L in lens]
    NB = sum(nbs) + 3
    perm = rng.permutation(np.arange(1, NB))
    kc = np.zeros((NB, KVH, 16, D), np.float16)
    vc = np.zeros_like(kc)
    width = max(nbs)
    bt = np.zeros((len(lens), width), np.int32)
    off = 0
    qs, ks, vs, qsl = [], [], [], [0]
    for b, (L, nb) in enumerate(zip(lens, nbs)):
        bt[b, :nb] = perm[off:off + nb]
        off += nb
        k, v = rnd((L, KVH, D), 100 + b), rnd((L, KVH, D), 200 + b)
        OP.kv_write(k, v, kc, vc, OP.slot_mapping(bt[b], np.arange(L)))
        ql = min(L, 3)
        qs.append(rnd((ql, H, D), 300 + b))
        ks.append(k)
        vs.append(v)
        qsl.append(qsl[-1] + ql)
    q = np.concatenate(qs)
    out = OP.paged_attention(q, kc, vc, qsl, lens, bt, 0.25, np.float64)
    for b in range(len(lens)):
        want = OP.attention_with_mask(qs[b], ks[b], vs[b], 0.25, np.float64)
        np.testing.assert_array_equal(out[qsl[b]:qsl[b + 1]], want)


def test_paged_zero_rows():
    H, KVH, D = 2, 1, 4
    kc, vc = rnd((4, KVH, 16, D), 1), rnd((4, KVH, 16, D), 2)
    q = rnd((3, H, D), 3)
    bt = np.array([[1], [2], [3]], np.int32)
    out = OP.paged_attention(q, kc, vc, [0, 1, 2, 3], [5, 0, 9], bt, 0.5)
    assert (out[1] == 0).all() and (out[0] != 0).any() and (out[2] != 0).any()


# ------------------------------------------------------------------------------------------
# split-K merge
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("L,P,splits", [(100, 16, 7), (100, 64, 4), (4096, 512, 8), (17, 512, 8),
                                        (33, 16, 3)])
def test_split_merge_equals_single_pass(L, P, splits):
    H, KVH, D = 6, 2, 8
    q, k, v = rnd((H, D), 1), rnd((L, KVH, D), 2), rnd((L, KVH, D), 3)
    m, l, a = OP.decode_partials(q, k, v, 0.35, P, splits)
    got = OP.split_merge(m, l, a)
    want = OP.attention_with_mask(q[None], k, v, 0.35, np.float64).reshape(H, D)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_split_merge_all_empty_is_zero():
    m = np.full((3, 4), -np.inf)
    l = np.zeros((3, 4))
    a = np.zeros((3, 4, 5))
    assert (OP.split_merge(m, l, a) == 0).all()


def test_split_merge_weights_by_max():
    """Two splits: one with a much larger max dominates; weights are exp(m_j - M)."""
    m = np.array([[0.0, 50.0]])
    l = np.array([[2.0, 1.0]])
    a = np.array([[[4.0], [3.0]]])
    assert np.allclose(OP.split_merge(m, l, a), [[3.0]])


# ------------------------------------------------------------------------------------------
# quantisation and the W8A16 product
# ------------------------------------------------------------------------------------------
def test_quantize_bounds_and_scale():
    w = np.random.default_rng(0).standard_normal((64, 96)).astype(np.float32) * 0.05
    w[3] = 0.0                                          # all-zero row: scale clamps to 1e-8
    wq, sc = OQ.quantize(w)
    assert wq.dtype == np.int8 and sc.dtype == np.float32
    assert wq.min() >= -127 and wq.max() <= 127
    assert np.allclose(sc[0], np.abs(w[0]).max() / 127) and sc[3] == np.float32(1e-8)
    assert (np.abs(np.abs(wq).max(axis=1)[np.arange(64) != 3] - 127) == 0).all()
    err = np.abs(OQ.dequantize(wq, sc) - w)
    assert (err <= sc[:, None] / 2 * (1 + 1e-6) + 1e-12).all()   # round-to-nearest bound


def test_round_half_even():
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -2.5]], np.float32)   # scale = 1
    wq, sc = OQ.quantize(w)
    assert sc[0] == 1.0 and wq.tolist() == [[127, 0, 2, 2, 0, -2]]


def test_w8a16_integer_closed_form():
    """scale = 1 and integer activations: the product is an exact integer matmul."""
    rng = np.random.default_rng(1)
    x = rng.integers(-8, 9, (5, 64)).astype(np.float16)
    wq = rng.integers(-127, 128, (12, 64)).astype(np.int8)
    y = OQ.w8a16(x, wq, np.ones(12, np.float32))
    assert np.array_equal(y, (x.astype(np.int64) @ wq.astype(np.int64).T).astype(np.float64))


def test_w8a16_gemv_loop_and_bias():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 40)).astype(np.float16)
    wq = rng.integers(-127, 128, (7, 40)).astype(np.int8)
    sc = rng.uniform(0.002, 0.02, 7).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float16)
    y = OQ.w8a16(x, wq, sc, b)
    for n in range(7):
        s = sum(float(x[0, kk]) * int(wq[n, kk]) for kk in range(40))
        assert abs(y[0, n] - (s * float(sc[n]) + float(b[n]))) < 1e-9


def test_linear_twin_close_to_exact():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 128)).astype(np.float16)
    wq, sc = OQ.quantize(rng.standard_normal((32, 128)).astype(np.float32) * 0.05)
    y = OQ.linear_twin(x, wq, sc).astype(np.float64)
    ref = OQ.w8a16(x, wq, sc)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-3
