"""numpy restatement of the paged-attention half of the hot path (test infrastructure only).

Arrays follow the reference layouts: q [T, H, D]; caches [num_blocks, KVH, 16, D];
block_tables [B, width] int32; seq_lens [B]; query_start_loc [B+1]; slot_mapping [T] int64.
``acc`` selects the accumulation dtype (float32 = the twins' arithmetic, float64 = exact-ish).
"""

from __future__ import annotations

import math

import numpy as np

BLOCK = 16


def slot_mapping(block_table, positions) -> np.ndarray:
    """slot(pos) = table[pos // 16] * 16 + pos % 16 (kv/kv_manager.py:39-40,
    runner/input_builder.py:59,123)."""
    bt = np.asarray(block_table, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    return bt[pos // BLOCK] * BLOCK + pos % BLOCK


def kv_write(k, v, k_cache, v_cache, slots) -> None:
    """In place: cache[slot // 16, :, slot % 16, :] = row, rows with slot < 0 skipped
    (ops/reference.py:50-57)."""
    slots = np.asarray(slots, dtype=np.int64)
    m = slots >= 0
    s = slots[m]
    k_cache[s // BLOCK, :, s % BLOCK, :] = k[m]
    v_cache[s // BLOCK, :, s % BLOCK, :] = v[m]


def gather(cache, table_row, seq_len: int) -> np.ndarray:
    """The first seq_len tokens of one sequence as [seq_len, KVH, D]
    (ops/reference.py:106-109: cache[blocks].permute(0, 2, 1, 3).reshape(nb * 16, KVH, D))."""
    nb = -(-seq_len // BLOCK)
    blocks = np.asarray(table_row[:nb], dtype=np.int64)
    g = cache[blocks]                                  # [nb, KVH, 16, D]
    return g.transpose(0, 2, 1, 3).reshape(nb * BLOCK, cache.shape[1], cache.shape[3])[:seq_len]


def attention_with_mask(q, k, v, scale: float, acc=np.float32) -> np.ndarray:
    """Masked GQA attention, q [Tq, H, D], k/v [Tk, KVH, D] -> [Tq, H * D] in ``acc``
    (ops/reference.py:60-77): each query head h reads KV head h // G; bottom-right causal mask
    j <= (Tk - Tq) + i; softmax over keys; no cast (callers round to fp16 where the twin does)."""
    Tq, H, D = q.shape
    Tk, KVH, _ = k.shape
    G = H // KVH
    qf = q.astype(acc).transpose(1, 0, 2)                              # [H, Tq, D]
    kf = np.repeat(k.astype(acc), G, axis=1).transpose(1, 0, 2)        # [H, Tk, D]
    vf = np.repeat(v.astype(acc), G, axis=1).transpose(1, 0, 2)
    scores = np.matmul(qf, kf.transpose(0, 2, 1)) * acc(scale)         # [H, Tq, Tk]
    i = np.arange(Tq)[:, None]
    j = np.arange(Tk)[None, :]
    scores = np.where(j <= (Tk - Tq) + i, scores, -np.inf)
    mx = scores.max(axis=-1, keepdims=True)
    p = np.exp(scores - mx)
    p = p / p.sum(axis=-1, keepdims=True)
    out = np.matmul(p, vf).transpose(1, 0, 2)                          # [Tq, H, D]
    return out.reshape(Tq, H * D)


def paged_attention(q, k_cache, v_cache, query_start_loc, seq_lens, block_tables, scale: float,
                    acc=np.float32) -> np.ndarray:
    """Ragged paged attention -> [T, H * D] in ``acc`` (ops/reference.py:94-111). Sequence b owns
    rows query_start_loc[b] .. query_start_loc[b+1]-1; rows of sequences with seq_len 0 or no
    query rows stay 0."""
    T, H, D = q.shape
    out = np.zeros((T, H * D), dtype=acc)
    qsl = [int(x) for x in query_start_loc]
    for b, seq_len in enumerate(int(x) for x in seq_lens):
        qs, qe = qsl[b], qsl[b + 1]
        if seq_len == 0 or qe == qs:
            continue
        kk = gather(k_cache, block_tables[b], seq_len)
        vv = gather(v_cache, block_tables[b], seq_len)
        out[qs:qe] = attention_with_mask(q[qs:qe], kk, vv, scale, acc)
    return out


def decode_partials(q_row, k, v, scale: float, partition: int, num_splits: int,
                    acc=np.float64):
    """Split-K partials of one decode row (ops/triton_decode_attention.py:101-141): split j covers
    tokens [j * P, min(j * P + P, seq_len)); returns m, l [H, splits] and acc [H, splits, D]
    with m = -inf, l = 0, acc = 0 for an empty split. q_row [H, D], k/v [seq_len, KVH, D]."""
    H, D = q_row.shape
    KVH = k.shape[1]
    G = H // KVH
    n = k.shape[0]
    m = np.full((H, num_splits), -np.inf, dtype=acc)
    l = np.zeros((H, num_splits), dtype=acc)
    a = np.zeros((H, num_splits, D), dtype=acc)
    for j in range(num_splits):
        lo, hi = j * partition, min(j * partition + partition, n)
        if hi <= lo:
            continue
        for h in range(H):
            kh = k[lo:hi, h // G].astype(acc)
            vh = v[lo:hi, h // G].astype(acc)
            s = kh @ q_row[h].astype(acc) * scale
            m[h, j] = s.max()
            p = np.exp(s - m[h, j])
            l[h, j] = p.sum()
            a[h, j] = p @ vh
    return m, l, a


def split_merge(m, l, a) -> np.ndarray:
    """Merge split partials (ops/triton_decode_attention.py:144-163): M = max_j m_j (0 if every
    split is empty), w_j = exp(m_j - M) (0 for an empty split), out = sum w_j acc_j / L with
    L = sum w_j l_j (1 if 0). m, l [..., S], a [..., S, D] -> [..., D]."""
    M = m.max(axis=-1, keepdims=True)
    M = np.where(np.isneginf(M), 0.0, M)
    with np.errstate(invalid="ignore"):
        w = np.where(np.isneginf(m), 0.0, np.exp(m - M))
    L = (l * w).sum(axis=-1)
    L = np.where(L == 0.0, 1.0, L)
    return (a * w[..., None]).sum(axis=-2) / L[..., None]


def attention_brute(q, k, v, scale: float) -> np.ndarray:
    """Pure-Python float64 loops (tiny inputs only): textbook softmax attention with the
    bottom-right causal mask, written independently of numpy's batched products."""
    Tq, H, D = q.shape
    Tk, KVH, _ = k.shape
    G = H // KVH
    out = np.zeros((Tq, H * D), dtype=np.float64)
    for i in range(Tq):
        for h in range(H):
            kvh = h // G
            scores = []
            for j in range(Tk):
                if j > (Tk - Tq) + i:
                    break
                s = 0.0
                for d in range(D):
                    s += float(q[i, h, d]) * float(k[j, kvh, d])
                scores.append(s * scale)
            if not scores:
                continue
            mx = max(scores)
            e = [math.exp(s - mx) for s in scores]
            tot = sum(e)
            for d in range(D):
                out[i, h * D + d] = sum(e[j] * float(v[j, kvh, d]) for j in range(len(e))) / tot
    return out
