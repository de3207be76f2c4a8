"""The LDS-tiled prefill paths (head_dim 128) against the oracle (needs an MI355X).

128-row query tiles share each staged 64-key step: the paired kernel (two units per workgroup,
stream-K key-range slots) or, when its slots would get few key steps, the 4-wavefront tile
kernel with its own split plan; split partials are combined by a merge kernel
(ts_prefill_attention_ws). Every form is checked against the oracle (ops/reference.py:60-77,
94-111) with the attention criterion of the other kernel tests, on shapes that put the diagonal,
the key tail and the split boundaries in every position of a step; a NaN-filled workspace and
NaN cache rows past seq_len must not reach the output. An odd GQA group (14 / 2, 28 / 4, as in
Qwen2-7B) puts the paired kernel in its two-tiles mode (256-row work items, 128-row units): the
same checks run there, unsplit, split and with understated bounds.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from turingserve_amd import _native as N
from turingserve_amd import hip_ops as K
from turingserve_amd import synth

from .test_kernels_gpu import DEV, assert_attn, make_paged, meta_of, oracle_attn

pytestmark = pytest.mark.gpu
H, KVH, D = 12, 2, 128


def run_prefill(q, kc, vc, qsl, sl, bt, meta, ws: torch.Tensor | None, ws_bytes: int | None = None,
                heads=(H, KVH)):
    H, KVH = heads
    out = torch.full((q.shape[0], H * D), float("nan"), dtype=torch.float16, device=DEV)
    B = sl.shape[0]
    common = (q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), q.shape[0],
              kc.data_ptr(), vc.data_ptr(), kc.shape[0], bt.data_ptr(), bt.stride(0), bt.shape[1],
              sl.data_ptr(), qsl.data_ptr(), B, meta.num_decode, int(meta.max_query_len))
    stream = torch.cuda.current_stream().cuda_stream
    if ws is None:
        N.check(N.lib().ts_prefill_attention(*common, H, KVH, D, D ** -0.5, stream), "prefill")
    else:
        nb = ws.numel() if ws_bytes is None else ws_bytes
        N.check(N.lib().ts_prefill_attention_ws(*common, int(meta.max_seq_len), H, KVH, D,
                                                D ** -0.5, ws.data_ptr(), nb, stream), "prefill")
    torch.cuda.synchronize()
    return out


def setup(q_lens, prefixes, seed=0, heads=(H, KVH)):
    seq = [p + n for p, n in zip(prefixes, q_lens)]
    q, kc, vc, qsl, sl, bt = make_paged(seq, heads[0], heads[1], D, list(q_lens), seed=seed)
    meta = meta_of(qsl, sl, bt, 0, list(q_lens), q.shape[0])
    dev = [x.to(DEV) for x in (q, kc, vc, qsl, sl, bt)]
    ref = oracle_attn(q, kc, vc, qsl, sl, bt, D ** -0.5)
    return dev, meta, ref


def ws_bytes_for(meta, P, heads=(H, KVH)):
    return N.lib().ts_prefill_workspace_bytes(P, heads[0], D, int(meta.max_query_len),
                                              int(meta.max_seq_len), N.cu_count(0))


@pytest.mark.parametrize("q_lens,prefixes", [
    ([1], [0]), ([63], [1]), ([128], [0]), ([129], [63]), ([200], [64]), ([512], [1037]),
    ([700], [3000]), ([2048], [0]), ([17], [4000]), ([5, 300, 128], [0, 900, 2500]),
    ([1024], [6000]), ([640, 512], [5000, 7000]),
])
def test_tiled_prefill_split_and_unsplit(q_lens, prefixes):
    """Without a workspace the paired kernel runs unsplit; with one, short key ranges per launch
    slot take the tile kernel's split plan and long ones (the last two cases) the paired
    kernel's stream-K plan."""
    (q, kc, vc, qsl, sl, bt), meta, ref = setup(q_lens, prefixes)
    out1 = run_prefill(q, kc, vc, qsl, sl, bt, meta, None)
    assert_attn(out1, ref, "unsplit")
    nb = ws_bytes_for(meta, len(q_lens))
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=DEV)
    out2 = run_prefill(q, kc, vc, qsl, sl, bt, meta, ws)
    assert_attn(out2, ref, "split")


@pytest.mark.parametrize("heads", [(14, 2), (28, 4)], ids=["14-2", "28-4"])
@pytest.mark.parametrize("q_lens,prefixes", [
    ([129], [63]), ([512], [1037]), ([700], [3000]), ([1024], [6000]),
    ([640, 512], [5000, 7000]),
])
def test_odd_group_prefill_split_and_unsplit(heads, q_lens, prefixes):
    """Odd GQA groups: the paired kernel's two-tiles mode unsplit (no workspace), and with a
    workspace the tile kernel's split plan (short key ranges per slot) or the paired kernel's
    stream-K plan merged by prefill_pair_merge_kernel (the long ones; the cases cover both
    routes for each group, test_odd_group_cases_cover_both_routes)."""
    (q, kc, vc, qsl, sl, bt), meta, ref = setup(q_lens, prefixes, seed=sum(q_lens), heads=heads)
    out1 = run_prefill(q, kc, vc, qsl, sl, bt, meta, None, heads=heads)
    assert_attn(out1, ref, f"unsplit {heads}")
    nb = ws_bytes_for(meta, len(q_lens), heads)
    assert nb > 0
    paired = _paired_route(int(meta.max_query_len), int(meta.max_seq_len), *heads, N.cu_count(0),
                           P=len(q_lens))
    ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
    out2 = run_prefill(q, kc, vc, qsl, sl, bt, meta, ws, heads=heads)
    assert_attn(out2, ref, f"split {heads} ({'stream-K' if paired else 'tile'})")


def test_odd_group_cases_cover_both_routes():
    cases = [([129], [63]), ([512], [1037]), ([700], [3000]), ([1024], [6000]),
             ([640, 512], [5000, 7000])]
    for heads in ((14, 2), (28, 4)):
        routes = {_paired_route(max(ql), max(p + n for p, n in zip(pf, ql)), *heads,
                                N.cu_count(0), P=len(ql)) for ql, pf in cases}
        assert routes == {True, False}, heads


def test_tiled_prefill_splits_when_it_should():
    """A short chunk on a long prefix gets a split plan (the case the split path is for), and a
    workspace one byte short of the queried size (a smaller plan, or none) gives the same
    result quality."""
    (q, kc, vc, qsl, sl, bt), meta, ref = setup([512], [1037], seed=3)
    nb = ws_bytes_for(meta, 1)
    assert nb > 0
    ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
    assert_attn(run_prefill(q, kc, vc, qsl, sl, bt, meta, ws, nb - 1), ref, "short workspace")
    assert_attn(run_prefill(q, kc, vc, qsl, sl, bt, meta, ws, nb), ref, "split")


def test_tiled_prefill_stale_nan_workspace():
    """Partials of empty splits and rows past q_len are never read: a NaN-filled workspace
    gives the same result."""
    (q, kc, vc, qsl, sl, bt), meta, ref = setup([300, 40], [1900, 333], seed=4)
    nb = ws_bytes_for(meta, 2)
    ws = torch.full((nb // 4 + 1,), float("nan"), dtype=torch.float32, device=DEV)
    out = run_prefill(q, kc, vc, qsl, sl, bt, meta, ws.view(torch.uint8), nb)
    assert_attn(out, ref, "nan workspace")


def test_tiled_prefill_nan_beyond_seq_len():
    """Cache rows past seq_len inside the last block hold NaN (a reused block): masked keys
    and zeroed V rows keep them out of the output."""
    q_lens, prefixes = [77], [250]           # seq_len 327: last block half used
    (q, kc, vc, qsl, sl, bt), meta, ref = setup(q_lens, prefixes, seed=6)
    seq = prefixes[0] + q_lens[0]
    last = int(bt[0, (seq - 1) // 16])
    kc[last, :, seq % 16:] = float("nan")
    vc[last, :, seq % 16:] = float("nan")
    out1 = run_prefill(q, kc, vc, qsl, sl, bt, meta, None)
    assert_attn(out1, ref, "nan tail unsplit")
    ws = torch.empty(max(ws_bytes_for(meta, 1), 16), dtype=torch.uint8, device=DEV)
    assert_attn(run_prefill(q, kc, vc, qsl, sl, bt, meta, ws), ref, "nan tail split")


def test_tiled_prefill_chunked_prompt_through_paged_attention():
    """A 3000-token prompt in 1024-token chunks (the shape of config 3, shortened so the oracle
    stays quick): each chunk's K/V written first, then paged_attention over the cache so far."""
    for ci, (prefix, n) in enumerate(synth.config3_chunks(prompt=3000, chunk=1024)):
        st = synth.config3(ci, seed=0, prompt=3000, chunk=1024)
        kc, vc = st.k_cache.to(DEV), st.v_cache.to(DEV)
        qkv = st.qkv.to(DEV)
        q, k, v = st.views(qkv)
        meta = st.meta(DEV)
        K.kv_write(k, v, kc, vc, meta.slot_mapping)
        out = K.paged_attention(q, kc, vc, meta, st.D ** -0.5)
        qn = q.float().cpu().half().numpy()
        ref = oracle_attn(torch.from_numpy(qn), kc.cpu(), vc.cpu(), meta.query_start_loc.cpu(),
                          meta.seq_lens.cpu(), meta.block_tables.cpu(), st.D ** -0.5)
        assert_attn(out, ref, f"chunk {ci} (prefix {prefix}, {n} rows)")


@pytest.mark.parametrize("D,n_decode,mql,q_len,prefix,heads", [
    (64, 0, 300, 600, 600, (12, 2)), (128, 0, 300, 600, 600, (12, 2)),
    (128, 0, 128, 600, 600, (12, 2)), (128, 4, 300, 600, 600, (12, 2)),
    (128, 0, 640, 1280, 8000, (12, 2)), (128, 0, 300, 600, 600, (14, 2)),
    (128, 0, 640, 1280, 8000, (14, 2))])
def test_understated_bounds_give_nan_rows_not_stale_memory(D, n_decode, mql, q_len, prefix, heads):
    """max_query_len below a chunk's real q_len (a caller bug): the rows the plan does not cover
    come out as NaN, the covered rows are still right.

    * head_dim 128, prefill only, few key steps per paired launch slot: the 4-wavefront tile
      kernel; tiles the launch misses (the lowest, launched longest first) are NaN.
    * head_dim 128, prefill only, many steps per slot: the paired kernel's stream-K plan shares
      the sequence's real steps over its launch slots, so every tile is computed; a tile whose
      segments run past the workspace the host bounds sized gets NaN rows. Tiles are numbered
      longest first, so those are the lowest tiles: the NaN rows are a tile-aligned prefix
      (128-row tiles with an even GQA group, 256-row ones with an odd group).
    * head_dim 128 with decode rows (one-launch ragged kernel): as the tile kernel.
    * head_dim < 128: the kernel covers rows from 0 up."""
    from turingserve_amd.metadata import AttentionMetadata

    Hh, KV = heads
    seq_len = prefix + q_len
    seq = [300 + 97 * i for i in range(n_decode)] + [seq_len]
    ql = [1] * n_decode + [q_len]
    q, kc, vc, qsl, sl, bt = make_paged(seq, Hh, KV, D, ql, seed=9)
    ref = oracle_attn(q, kc, vc, qsl, sl, bt, D ** -0.5)
    dq, dkc, dvc, dqsl, dsl, dbt = (x.to(DEV) for x in (q, kc, vc, qsl, sl, bt))
    T = n_decode + q_len
    meta = AttentionMetadata(dqsl, dsl, dbt, torch.zeros(T, dtype=torch.int64, device=DEV),
                             n_decode, mql, seq_len)           # max_query_len understated
    out = K.paged_attention(dq, dkc, dvc, meta, D ** -0.5)
    torch.cuda.synchronize()
    o = out.float().cpu()[n_decode:]
    nan_rows = torch.isnan(o).all(dim=1)
    rows_i = torch.arange(q_len)
    tiles = -(-q_len // 128)
    cus = N.cu_count(0)
    paired = D == 128 and n_decode == 0 and _paired_route(mql, seq_len, Hh, KV, cus)
    assert paired == (prefix == 8000), "the cases cover each route once"
    if paired:
        tr = 128 if (Hh // KV) % 2 == 0 else 256
        covered = rows_i >= tr * _stream_k_nan_tiles(mql, q_len, seq_len, Hh, KV, cus)
    elif D == 128:
        covered = rows_i >= 128 * (tiles - (-(-mql // 128)))   # the longest cdiv(mql, 128) tiles
    else:
        covered = rows_i < 32 * (-(-mql // 32))                 # tiles of 32 rows from row 0
    assert bool(nan_rows[~covered].all()) and not bool(torch.isnan(o[covered]).any())
    rows = torch.cat([torch.ones(n_decode, dtype=torch.bool), covered])
    assert_attn(out[rows.to(DEV)], ref[rows.numpy()], f"covered rows, D {D}")


def _pair_shape(H: int, KVH: int) -> tuple[int, int]:
    """(rows per work item, work items per sequence) of the paired kernel: two query heads of
    128 rows with an even GQA group, two 128-row tiles of one head with an odd group."""
    return (128, H // 2) if (H // KVH) % 2 == 0 else (256, H)


def _paired_route(mql: int, msl: int, H: int, KVH: int, cus: int, P: int = 1) -> bool:
    """Whether a prefill-only head_dim 128 launch with a workspace takes the paired kernel: its
    stream-K plan gives each of the cus // items slots of a work item at least 16 of the
    cdiv(mql, tr) * cdiv(msl, 64) key steps the host bounds allow."""
    tr, items = _pair_shape(H, KVH)
    slots = cus // (items * P)
    return -(-mql // tr) * -(-max(msl, mql) // 64) >= 16 * slots


def _stream_k_nan_tiles(mql: int, q_len: int, seq_len: int, H: int, KVH: int, cus: int) -> int:
    """Lowest 128-row tiles (two heads per work item) of one prefill sequence that the stream-K
    plan sized for max_query_len = mql leaves as NaN: tiles, longest first, share the sequence's
    steps over `slots` launch slots; the tile at position pos with segments pos + k,
    k = G // T .. (G + n - 1) // T, is NaN when it has more than one segment and one of them is
    past the workspace's tiles_h + slots segments."""
    tr, items = _pair_shape(H, KVH)
    slots = cus // items
    seg_cap = -(-mql // tr) + slots
    tiles = -(-q_len // tr)
    prefix = seq_len - q_len
    steps = [-(-min(prefix + min((t + 1) * tr, q_len), seq_len) // 64) for t in range(tiles)]
    per = -(-sum(steps) // slots)
    nan, g = [], 0
    for pos in range(tiles):
        t = tiles - 1 - pos
        k0, k1 = g // per, (g + steps[t] - 1) // per
        nan.append(k0 < k1 and pos + k1 >= seg_cap)
        g += steps[t]
    # the NaN tiles must be the lowest ones (a row prefix)
    flags = [nan[tiles - 1 - t] for t in range(tiles)]
    n = 0
    while n < tiles and flags[n]:
        n += 1
    assert not any(flags[n:]), flags
    return n
