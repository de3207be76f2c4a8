"""The per-step decode split map (ts_decode_split_map; needs an MI355X).

The map is this library's own schedule table (the reference's fixed split grid needs no lookup,
ops/triton_decode_attention.py:187-200), so it is pinned two ways: its entries against a
restatement of the split schedule written from the rule the kernel documents (dense split
numbering in sequence order; by default a sequence of nb blocks cut into
n = min(max_splits, ceil(nb / 24)) splits of P = ceil(nb / n) rounded up to 8 blocks, its own
length alone deciding; fixed partitions capped at the launched grid), and every decode call that
reads it against the same call without it, bit for bit: outputs and caches (the attention
arithmetic is unchanged, only where a workgroup learns its split from). A map built for another
plan must be ignored, a map too small for the plan rejected, and a map built for another step
(other lengths, same plan) must poison the rows it would attend wrongly.
"""

from __future__ import annotations

import pytest
import torch

from turingserve_amd import _native as N
from turingserve_amd import hip_ops as K
from turingserve_amd import synth

from .test_decode_kv_write_gpu import decode_step, meta_for, rope_tables, views
from .test_kernels_gpu import DEV

pytestmark = pytest.mark.gpu

HEADER, ENTRY, MAGIC = 8, 32, 0x314D5354


OWN_PART = 24                                   # the own-length schedule's longest split


def own_part(nb, max_splits):
    """P_s of the own-length schedule for a sequence of nb blocks."""
    n = min(max(-(-nb // OWN_PART), 1), max_splits)
    return max(8, (-(-nb // n) + 7) // 8 * 8)


def expected_entries(lens, bt, NB, nslots, part_blocks, max_splits, cap_blocks):
    """The map entries of the schedule, one list of 32 ints per launch slot."""
    cap = cap_blocks * 16
    L = [min(max(int(x), 0), cap) for x in lens]
    nb = [(x + 15) // 16 for x in L]
    clamp = lambda b: b if 0 <= b < NB else 0
    ent, first = [], 0
    for i, nbi in enumerate(nb):
        ps = own_part(nbi, max_splits) if part_blocks <= 0 else part_blocks
        n = -(-nbi // ps) if nbi > 0 else 1     # a padding row still gets one (zero) split
        for j in range(n):
            lo, hi = j * ps, min(j * ps + ps, nbi)
            npairs = (hi - lo + 1) // 2
            ids = []
            for q in range(8):              # pairs 0..7: wavefront q % 4's first two pairs
                qq = q if q < npairs else (q - 4 if q >= 4 else q)
                ids += [clamp(int(bt[i, min(lo + 2 * qq + h, hi - 1)])) if nbi > 0 else 0
                        for h in range(2)]
            last = clamp(int(bt[i, (L[i] - 1) // 16])) if L[i] > 0 else 0
            ent.append([i, first, n, L[i], lo, hi, last, ps] + ids + [0] * 8)
        first += n
    assert len(ent) <= nslots
    return ent + [[-1] + [0] * 31] * (nslots - len(ent))


def abi_decode(q, kc, vc, meta, H, KVH, D, scale, smap, version="v3", partition=0):
    """ts_decode_attention on the step's caches, with the split map smap (or none)."""
    bt_d, sl_d = meta.block_tables.to(torch.int32), meta.seq_lens.to(torch.int32)
    S = sl_d.shape[0]
    code, part = K._decode_plan(S, int(meta.max_seq_len), version, partition)
    wsb = N.lib().ts_decode_workspace_bytes(code, S, H, KVH, D, int(meta.max_seq_len), part,
                                            N.cu_count(0))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    o = torch.empty(S, H * D, dtype=torch.float16, device=DEV)
    ptr, nb = (None, 0) if smap is None else (smap[0].data_ptr(), smap[1])
    N.check(N.lib().ts_decode_attention(
        code, q.data_ptr(), q.stride(0), q.stride(1), o.data_ptr(), o.stride(0),
        kc.data_ptr(), vc.data_ptr(), kc.shape[0], bt_d.data_ptr(), bt_d.stride(0),
        bt_d.shape[1], sl_d.data_ptr(), S, H, KVH, D, scale, int(meta.max_seq_len), part,
        ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream, ptr, nb), "decode")
    return o


def build(meta, H, KVH, D, NB, version=None, partition=None):
    return K.decode_split_map(meta, H, KVH, D, NB, torch.device(DEV), decode_version=version,
                              partition=partition)


def cases():
    g = torch.Generator().manual_seed(11)
    c2 = synth.config2(seed=1)
    mixed = synth.log_uniform_ints(40, 1, 3000, g)
    mixed[0], mixed[5], mixed[6] = 1, 16, 17
    return {
        "config2": [int(x) for x in c2.seq_lens],
        "mixed": mixed,
        "long_one": [32768, 40, 700, 5],        # 2048 blocks over 32 splits: P_s grows to 64
        "few": [4000, 2500],
    }


@pytest.mark.parametrize("name", ["config2", "mixed", "long_one", "few"])
@pytest.mark.parametrize("version,partition", [("v3", 0), ("v3", 256), (None, None)])
def test_map_entries_follow_the_schedule(name, version, partition):
    H, KVH, D = 12, 2, 128
    lens = cases()[name]
    qkv, kc, vc, qsl, sl, bt, slots = decode_step(lens, H, KVH, D, seed=len(lens))
    meta = meta_for(qsl, sl, bt, slots)
    if name == "long_one":
        meta.max_seq_len = 4096              # a host bound below the longest context
    NB = kc.shape[0]
    sm = build(meta, H, KVH, D, NB, version, partition)
    if sm is None:
        pytest.skip("this plan does not split")
    buf, nbytes = sm
    torch.cuda.synchronize()
    m = buf.cpu().tolist()
    groups = KVH * -(-(H // KVH) // 16)
    nslots = (nbytes // 4 - HEADER - len(lens) * groups) // ENTRY
    assert m[0] == MAGIC and m[1] == len(lens) and m[2] == nslots
    part_blocks, max_splits, cap = m[3], m[5], m[6]
    assert m[4] == 0 and m[7] == 0
    if part_blocks > 0:                      # the fixed grid covers ceil(max_seq_len / partition)
        max_blk = -(-int(meta.max_seq_len) // 16)
        assert cap == min(-(-max_blk // part_blocks) * part_blocks, bt.shape[1])
    else:
        assert cap == bt.shape[1]
    want = expected_entries(lens, bt, NB, nslots, part_blocks, max_splits, cap)
    got = [m[HEADER + s * ENTRY: HEADER + (s + 1) * ENTRY] for s in range(nslots)]
    for s in range(nslots):
        assert got[s] == want[s], f"slot {s}: {got[s]} != {want[s]}"
    # the arrival counters of the in-launch merge follow the entries, all zero
    assert m[HEADER + nslots * ENTRY:] == [0] * (len(lens) * groups)


@pytest.mark.parametrize("name", ["config2", "mixed", "long_one", "long_one_capped"])
@pytest.mark.parametrize("version,partition", [(None, None), ("v3", 256)])
def test_decode_with_map_equals_without(name, version, partition):
    H, KVH, D = 12, 2, 128
    lens = cases()[name.replace("_capped", "")]
    case = decode_step(lens, H, KVH, D, seed=7, pad=(1,))
    qkv, kc, vc, qsl, sl, bt, slots = case
    meta = meta_for(qsl, sl, bt, slots)
    if name.endswith("_capped"):
        meta.max_seq_len = 4096            # the fixed grid then covers 4096 of the 32768 tokens
    NB = kc.shape[0]
    q, k, v = views(qkv.to(DEV), H, KVH, D)
    scale = D ** -0.5
    sm = build(meta, H, KVH, D, NB, version, partition)
    assert sm is not None
    outs, caches = [], []
    for smap in (None, sm):
        kc1, vc1 = kc.to(DEV), vc.to(DEV)
        outs.append(K.decode_kv_write_attention(q, k, v, kc1, vc1, meta, scale,
                                                decode_version=version, partition=partition,
                                                split_map=smap))
        caches.append((kc1, vc1))
    torch.cuda.synchronize()
    # bit for bit; a capped grid leaves the longest sequence's fused write unsatisfiable (its
    # position is past the grid), so that row is NaN, alike with and without the map
    same = lambda a, b: torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True)  # noqa: E731
    same(outs[0], outs[1])
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    # the attention call alone through the C ABI (ts_decode_attention), with and without it
    bt_d, sl_d = meta.block_tables.to(torch.int32), meta.seq_lens.to(torch.int32)
    S = len(lens)
    code, part = K._decode_plan(S, int(meta.max_seq_len), version, partition)
    wsb = N.lib().ts_decode_workspace_bytes(code, S, H, KVH, D, int(meta.max_seq_len), part,
                                            N.cu_count(0))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    kcw, vcw = caches[0]
    res = []
    for ptr, nb in ((None, 0), (sm[0].data_ptr(), sm[1])):
        o = torch.empty(S, H * D, dtype=torch.float16, device=DEV)
        N.check(N.lib().ts_decode_attention(
            code, q.data_ptr(), q.stride(0), q.stride(1), o.data_ptr(), o.stride(0),
            kcw.data_ptr(), vcw.data_ptr(), NB, bt_d.data_ptr(), bt_d.stride(0), bt_d.shape[1],
            sl_d.data_ptr(), S, H, KVH, D, scale, int(meta.max_seq_len), part, ws.data_ptr(), wsb,
            torch.cuda.current_stream().cuda_stream, ptr, nb), "decode")
        res.append(o)
    torch.cuda.synchronize()
    same(res[0], res[1])
    if not name.endswith("_capped"):
        same(res[0], outs[0])


def test_rope_fused_decode_with_map():
    H, KVH, D = 12, 2, 128
    lens = cases()["mixed"]
    qkv, kc, vc, qsl, sl, bt, slots = decode_step(lens, H, KVH, D, seed=9, pad=(3,))
    meta = meta_for(qsl, sl, bt, slots)
    cos, sin = rope_tables(D, 3000)
    pos = (sl.long() - 1).clamp(min=0).to(DEV)
    sm = build(meta, H, KVH, D, kc.shape[0])
    assert sm is not None
    outs, caches = [], []
    for smap in (None, sm):
        kc1, vc1 = kc.to(DEV), vc.to(DEV)
        outs.append(K.decode_rope_kv_write_attention(qkv.to(DEV), pos, cos, sin, H, KVH, D, kc1,
                                                     vc1, meta, D ** -0.5, split_map=smap))
        caches.append((kc1, vc1))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])


def test_map_of_another_plan_poisons_and_a_short_map_is_rejected():
    """A launch given a map merges its splits in-launch (no merge kernel follows), so a map
    whose header names another plan cannot be ignored: every row comes out NaN, loudly. A map
    smaller than the plan needs is rejected before anything is launched."""
    H, KVH, D = 12, 2, 128
    lens = cases()["config2"]
    qkv, kc, vc, qsl, sl, bt, slots = decode_step(lens, H, KVH, D, seed=3)
    meta = meta_for(qsl, sl, bt, slots)
    NB = kc.shape[0]
    q, k, v = views(qkv.to(DEV), H, KVH, D)
    scale = D ** -0.5
    fixed = build(meta, H, KVH, D, NB, "v3", 256)       # 64 x 16 slots
    own = build(meta, H, KVH, D, NB, "v3", 0)           # 64 x ceil(max blocks / 24) slots
    assert fixed[1] > own[1]
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    ref = K.decode_kv_write_attention(q, k, v, kc1, vc1, meta, scale, decode_version="v3",
                                      partition=0)
    kc2, vc2 = kc.to(DEV), vc.to(DEV)
    out = K.decode_kv_write_attention(q, k, v, kc2, vc2, meta, scale, decode_version="v3",
                                      partition=0, split_map=fixed)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all() and torch.isnan(out).all()
    with pytest.raises(ValueError, match="split map"):
        K.decode_kv_write_attention(q, k, v, kc.to(DEV), vc.to(DEV), meta, scale,
                                    decode_version="v3", partition=256, split_map=own)


@pytest.mark.parametrize("fused", [False, True])
def test_map_of_the_previous_step_poisons_the_rows_it_would_misread(fused):
    """A map is built from one step's seq_lens and block tables. Passed to a later step of the
    same batch size (same plan, so the header matches), every row whose length moved on comes
    out NaN instead of being attended with the old split ranges; rows whose length did not move
    are unaffected and equal the map-free call."""
    H, KVH, D = 12, 2, 128
    lens = cases()["config2"]
    qkv, kc, vc, qsl, sl, bt, slots = decode_step(lens, H, KVH, D, seed=5)
    meta = meta_for(qsl, sl, bt, slots)
    NB = kc.shape[0]
    q, k, v = views(qkv.to(DEV), H, KVH, D)
    scale = D ** -0.5
    moved = [i % 3 != 0 for i in range(len(lens))]      # two rows in three advanced one token
    prev = [x - 1 if m else x for x, m in zip(lens, moved)]
    meta_prev = meta_for(qsl, torch.tensor(prev, dtype=sl.dtype), bt, slots)
    meta_prev.max_seq_len = meta.max_seq_len                 # the same plan as this step's
    stale = build(meta_prev, H, KVH, D, NB, "v3", 0)
    fresh = build(meta, H, KVH, D, NB, "v3", 0)
    assert stale is not None and stale[1] == fresh[1]
    res = {}
    for name, smap in (("none", None), ("fresh", fresh), ("stale", stale)):
        kc1, vc1 = kc.to(DEV), vc.to(DEV)
        if fused:
            res[name] = K.decode_kv_write_attention(q, k, v, kc1, vc1, meta, scale,
                                                    decode_version="v3", partition=0,
                                                    split_map=smap)
        else:                                    # the attention call alone, through the C ABI
            K.kv_write(k, v, kc1, vc1, meta.slot_mapping)
            res[name] = abi_decode(q, kc1, vc1, meta, H, KVH, D, scale, smap)
    torch.cuda.synchronize()
    assert torch.equal(res["fresh"], res["none"])
    assert torch.isfinite(res["none"]).all()
    for i, m in enumerate(moved):
        row = res["stale"][i]
        if m:
            assert torch.isnan(row).all(), f"row {i} (moved) attended with a stale map"
        else:
            assert torch.equal(row, res["none"][i]), f"row {i} (unmoved) changed"


def test_map_built_inside_graph_replays():
    """The map build and the layers' fused calls captured in one graph, as a model step is:
    every replay (with eager work between them) equals the eager calls without a map."""
    st = synth.config2(seed=4)
    qkv = st.qkv.to(DEV)
    q, k, v = st.views(qkv)
    meta = st.meta(DEV)
    meta.in_graph = True
    scale = st.D ** -0.5
    NB = st.k_cache.shape[0]
    kc, vc = st.k_cache.to(DEV), st.v_cache.to(DEV)
    ref = K.decode_kv_write_attention(q, k, v, kc, vc, meta, scale)
    layers = [(st.k_cache.to(DEV), st.v_cache.to(DEV)) for _ in range(2)]
    outs = []
    sm = build(meta, st.H, st.KVH, st.D, NB)        # eager first: library and allocator warm
    for kcl, vcl in layers:
        K.decode_kv_write_attention(q, k, v, kcl, vcl, meta, scale, split_map=sm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sm = build(meta, st.H, st.KVH, st.D, NB)
        for kcl, vcl in layers:
            outs.append(K.decode_kv_write_attention(q, k, v, kcl, vcl, meta, scale, split_map=sm))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(o, ref)
        scratch = torch.randn(1 << 20, device=DEV).sum()
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
    for kcl, vcl in layers:
        assert torch.equal(kcl, kc) and torch.equal(vcl, vc)
