"""The ``hip`` op namespace: the reference's op signatures on the gfx950 kernels.

Mirrors ops/triton_ops.py (dispatch, decode-version selection, linear routing),
ops/triton_kv_write.py:28-35, ops/triton_decode_attention.py:169-200,
ops/triton_prefill_attention.py:66-79, ops/triton_w8a16.py:38-51 and the fused small ops
(ops/triton_rmsnorm.py:30-46, ops/triton_rope.py:27-31, ops/triton_silu_mul.py:21-28). Every op turns its tensors
into pointers and strides, allocates outputs and scratch from the torch caching allocator (so the
calls can be captured into a hipGraph) and launches on torch's current stream. A shape the
kernels do not support raises ValueError; nothing falls back to another implementation.

Triton tuning knobs the reference's launch helpers accept (block_n, num_warps, num_stages,
block_m) are accepted and ignored: the HIP kernels fix their own tile shapes.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from turingserve_amd import _native as N
from turingserve_amd import tuner
from turingserve_amd.quant import LinearWeight

__all__ = ["kv_write", "paged_attention", "linear", "lm_head_int8", "logits_int8", "w8a16_linear",
           "decode_attention_v1", "decode_attention_v2", "decode_attention_v3",
           "prefill_attention", "rmsnorm", "rmsnorm_residual", "rope_", "silu_mul", "w8a16_glu",
           "gate_up_silu", "rope_kv_write_", "decode_kv_write_attention",
           "decode_rope_kv_write_attention"]

DEFAULT_PARTITION = 0            # v3 split size when the caller names none: 0 = own-length


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        _require(t.is_cuda, "hip backend: every tensor must live on the GPU")


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[int, int, int]:
    _require(k_cache.dim() == 4 and k_cache.shape[2] == 16 and k_cache.shape == v_cache.shape,
             f"caches must be [num_blocks, KVH, 16, D], got {tuple(k_cache.shape)}")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    _require(k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16,
             "hip backend: the KV cache must be fp16")
    NB, KVH, _, D = k_cache.shape
    return NB, KVH, D


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.int32 and t.is_contiguous()) else t.to(torch.int32).contiguous()


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    return None if nbytes == 0 else torch.empty(nbytes, dtype=torch.uint8, device=device)


# ------------------------------------------------------------------------------------------
# kv_write (ops/triton_kv_write.py:28-35)
# ------------------------------------------------------------------------------------------
def kv_write(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             slot_mapping: torch.Tensor) -> None:
    """k, v: [T, KVH, D] (strided views of qkv allowed); caches [NB, KVH, 16, D]."""
    T, KVH, D = k.shape
    if T == 0:
        return
    _check_gpu(k, v, k_cache, v_cache, slot_mapping)
    NB, ckvh, cd = _check_cache(k_cache, v_cache)
    _require(v.shape == k.shape and ckvh == KVH and cd == D, "kv_write: shape mismatch")
    _require(k.dtype == torch.float16 and v.dtype == torch.float16, "kv_write: k, v must be fp16")
    _require(k.stride(2) == 1 and v.stride(2) == 1, "kv_write: head_dim must be unit-stride")
    _require(slot_mapping.shape[0] >= T, "kv_write: slot_mapping shorter than k")
    slots = slot_mapping if (slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous()) \
        else slot_mapping.to(torch.int64).contiguous()
    N.check(N.lib().ts_kv_write(_ptr(k), _ptr(v), k.stride(0), k.stride(1), v.stride(0),
                                v.stride(1), _ptr(k_cache), _ptr(v_cache), NB, _ptr(slots), T,
                                KVH, D, _stream(k)), "kv_write")


# ------------------------------------------------------------------------------------------
# decode (ops/triton_ops.py:35-57, ops/triton_decode_attention.py:169-200)
# ------------------------------------------------------------------------------------------
def _decode_call(version: int, q, out, k_cache, v_cache, block_tables, seq_lens, scale: float,
                 S: int, max_seq_len: int, partition: int) -> None:
    if S == 0:
        return
    _check_gpu(q, out, k_cache, v_cache, block_tables, seq_lens)
    NB, KVH, D = _check_cache(k_cache, v_cache)
    _, H, qd = q.shape
    _require(qd == D and q.stride(2) == 1 and q.dtype == torch.float16,
             "decode: q must be fp16 [T, H, D] with unit stride over D")
    _require(out.stride(1) == 1 and out.dtype == torch.float16, "decode: out must be fp16 rows")
    bt = _i32(block_tables)
    sl = _i32(seq_lens)
    dev = q.device
    cus = N.cu_count(dev.index or 0)
    ws_bytes = N.lib().ts_decode_workspace_bytes(version, S, H, KVH, D, max_seq_len, partition, cus)
    ws = _workspace(ws_bytes, dev)
    N.check(N.lib().ts_decode_attention(
        version, _ptr(q), q.stride(0), q.stride(1), _ptr(out), out.stride(0), _ptr(k_cache),
        _ptr(v_cache), NB, _ptr(bt), bt.stride(0), bt.shape[1], _ptr(sl), S, H, KVH, D,
        float(scale), int(max_seq_len), int(partition), _ptr(ws), ws_bytes, _stream(q), None, 0),
        "decode_attention")


def _decode_plan(S: int, max_seq_len: int, decode_version: str | None,
                 partition: int | None) -> tuple[int, int]:
    """(version code, partition) of a fused decode call: the variant table's choice for
    (S, max_seq_len) when no version is given, the default partition for v3 / AUTO."""
    _require(decode_version in N.DECODE_VERSIONS, f"unknown decode version {decode_version!r}")
    if decode_version is None:
        tv, tp = tuner.decode_choice(S, int(max_seq_len))
        if tv is not None:
            decode_version = tv
            partition = tp if partition is None else partition
    code = N.DECODE_VERSIONS[decode_version]
    part = (DEFAULT_PARTITION if partition is None else partition) if code in (0, 3) else 0
    return code, part


def _map_args(split_map) -> tuple:
    return (None, 0) if split_map is None else (_ptr(split_map[0]), split_map[1])


def decode_split_map(meta, H: int, KVH: int, D: int, num_blocks: int, device,
                     decode_version: str | None = None, partition: int | None = None):
    """The step's split map (ts_decode_split_map) for the fused decode calls of a pure-decode
    step with this attention shape: built once, passed as split_map= to every layer's
    decode_kv_write_attention / decode_rope_kv_write_attention of the same step (same meta,
    decode_version and partition). Returns (int32 device tensor, bytes), or None when the plan
    does not split (nothing to build; the calls then take split_map=None)."""
    S = meta.num_decode
    if S == 0:
        return None
    code, part = _decode_plan(S, int(meta.max_seq_len), decode_version, partition)
    nb = N.lib().ts_decode_split_map_bytes(code, S, H, KVH, D, int(meta.max_seq_len), part,
                                          N.cu_count(device.index or 0))
    if nb == 0:
        return None
    bt, sl = _i32(meta.block_tables), _i32(meta.seq_lens)
    _check_gpu(bt, sl)
    buf = torch.empty(nb // 4, dtype=torch.int32, device=device)
    N.check(N.lib().ts_decode_split_map(code, _ptr(bt), bt.stride(0), bt.shape[1], int(num_blocks),
                                        _ptr(sl), S, H, KVH, D, int(meta.max_seq_len), part,
                                        _ptr(buf), nb, _stream(buf)), "decode_split_map")
    return buf, nb


def decode_attention_v1(q, out, k_cache, v_cache, block_tables, seq_lens, scale, S: int):
    """One wavefront per (sequence, query head) (ops/triton_decode_attention.py:169-174)."""
    _decode_call(1, q, out, k_cache, v_cache, block_tables, seq_lens, scale, S, 0, 0)


def decode_attention_v2(q, out, k_cache, v_cache, block_tables, seq_lens, scale, S: int,
                        block_n: int = 32, num_warps: int = 4):
    """One workgroup per (sequence, KV head) (ops/triton_decode_attention.py:177-184)."""
    _decode_call(2, q, out, k_cache, v_cache, block_tables, seq_lens, scale, S, 0, 0)


def decode_attention_v3(q, out, k_cache, v_cache, block_tables, seq_lens, scale, S: int,
                        num_splits: int, partition: int = 512, block_n: int = 32,
                        num_warps: int = 4):
    """Split-K over `num_splits` partitions of `partition` tokens + merge
    (ops/triton_decode_attention.py:187-200)."""
    _decode_call(3, q, out, k_cache, v_cache, block_tables, seq_lens, scale, S,
                 num_splits * partition, partition)


def _decode(q, out, k_cache, v_cache, meta, scale, version: str | None = None):
    """Decode rows [0, num_decode) of the batch (ops/triton_ops.py:35-57). version None lets the
    library choose: own-length split-K when one workgroup per (sequence, KV head) would leave CUs
    idle and contexts exceed 256 tokens, else one workgroup per (sequence, KV head)."""
    _require(version in N.DECODE_VERSIONS, f"unknown decode version {version!r}")
    S = meta.num_decode
    code = N.DECODE_VERSIONS[version]
    part = DEFAULT_PARTITION if code in (0, 3) else 0
    _decode_call(code, q, out, k_cache, v_cache, meta.block_tables, meta.seq_lens, scale, S,
                 meta.max_seq_len, part)


# ------------------------------------------------------------------------------------------
# prefill (ops/triton_prefill_attention.py:66-79)
# ------------------------------------------------------------------------------------------
def prefill_attention(q, out, k_cache, v_cache, meta, scale, block_m: int = 64,
                      block_n: int = 64, num_warps: int = 4, num_stages: int = 2):
    """Sequences num_decode .. B-1 of the batch; q [T, H, D] flat, out [T, H*D]."""
    B = meta.seq_lens.shape[0]
    if B <= meta.num_decode:
        return
    _check_gpu(q, out, k_cache, v_cache)
    NB, KVH, D = _check_cache(k_cache, v_cache)
    T, H, qd = q.shape
    _require(qd == D and q.stride(2) == 1 and q.dtype == torch.float16,
             "prefill: q must be fp16 [T, H, D] with unit stride over D")
    bt, sl, qsl = _i32(meta.block_tables), _i32(meta.seq_lens), _i32(meta.query_start_loc)
    ws_bytes = _prefill_ws_bytes(B - meta.num_decode, H, D, meta, q.device)
    ws = _workspace(ws_bytes, q.device)
    N.check(N.lib().ts_prefill_attention_ws(
        _ptr(q), q.stride(0), q.stride(1), _ptr(out), out.stride(0), T, _ptr(k_cache),
        _ptr(v_cache), NB, _ptr(bt), bt.stride(0), bt.shape[1], _ptr(sl), _ptr(qsl), B,
        meta.num_decode, int(meta.max_query_len), _prefill_seq_bound(meta), H, KVH, D,
        float(scale), _ptr(ws), ws_bytes, _stream(q)), "prefill_attention")


def _prefill_ws_bytes(P: int, H: int, D: int, meta, device) -> int:
    """Workspace of the split prefill path (0 when the batch has no prefill rows)."""
    if P <= 0:
        return 0
    return N.lib().ts_prefill_workspace_bytes(P, H, D, int(meta.max_query_len),
                                              _prefill_seq_bound(meta), N.cu_count(device.index or 0))


def _prefill_seq_bound(meta) -> int:
    """Host bound of the prefill rows' seq_lens (the builders record it; else max_seq_len)."""
    b = int(getattr(meta, "max_prefill_seq_len", 0) or 0)
    return b if b > 0 else int(meta.max_seq_len)


# ------------------------------------------------------------------------------------------
# paged_attention (ops/triton_ops.py:60-71)
# ------------------------------------------------------------------------------------------
def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, meta,
                    scale: float, decode_version: str | None = None,
                    partition: int | None = None) -> torch.Tensor:
    """q [T, H, D] -> [T, H*D]: decode kernel on rows [0, num_decode), prefill kernel on the
    remaining sequences, one library call. Unless the caller names a decode version, the active
    variant table's choice for (num_decode, max_seq_len) applies to a pure-decode batch (the
    workload the table times), then the library's own policy with the own-length split
    (partition 0), which a mixed batch always takes: only that plan runs its decode rows and
    prefill tiles in one launch (a tuned fixed partition made the config 5 mixed step 4.13 ->
    4.60 ms by splitting the call in two)."""
    T, H, D = q.shape
    out = torch.empty(T, H * D, dtype=q.dtype, device=q.device)
    if T == 0:
        return out
    _check_gpu(q, k_cache, v_cache)
    NB, KVH, cd = _check_cache(k_cache, v_cache)
    _require(cd == D and q.stride(2) == 1 and q.dtype == torch.float16,
             "paged_attention: q must be fp16 [T, H, D] with unit stride over D")
    _require(decode_version in N.DECODE_VERSIONS, f"unknown decode version {decode_version!r}")
    bt, sl, qsl = _i32(meta.block_tables), _i32(meta.seq_lens), _i32(meta.query_start_loc)
    B = sl.shape[0]
    S = meta.num_decode
    if decode_version is None and S > 0 and B == S:
        tv, tp = tuner.decode_choice(S, int(meta.max_seq_len))
        if tv is not None:
            decode_version = tv
            partition = tp if partition is None else partition
    partition = DEFAULT_PARTITION if partition is None else partition
    code = N.DECODE_VERSIONS[decode_version]
    ws_bytes = N.lib().ts_paged_attention_workspace_bytes(
        B, S, int(meta.max_query_len), int(meta.max_seq_len), _prefill_seq_bound(meta), H, KVH, D,
        code, int(partition), N.cu_count(q.device.index or 0))
    ws = _workspace(ws_bytes, q.device)
    N.check(N.lib().ts_paged_attention(
        _ptr(q), q.stride(0), q.stride(1), _ptr(out), out.stride(0), T, _ptr(k_cache),
        _ptr(v_cache), NB, _ptr(bt), bt.stride(0), bt.shape[1], _ptr(sl), _ptr(qsl), B, S,
        int(meta.max_query_len), int(meta.max_seq_len), _prefill_seq_bound(meta), H, KVH, D,
        float(scale), code,
        int(partition), _ptr(ws), ws_bytes, _stream(q)), "paged_attention")
    return out


def decode_kv_write_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              k_cache: torch.Tensor, v_cache: torch.Tensor, meta, scale: float,
                              decode_version: str | None = None,
                              partition: int | None = None, split_map=None) -> torch.Tensor:
    """A pure-decode layer step in one launch: kv_write(k, v, caches, meta.slot_mapping) and
    then paged_attention(q, caches, meta, scale) (model/qwen2.py:26-28 with
    ops/triton_ops.py:60-71), returning the same [T, H*D] and leaving the same cache. q [T, H, D],
    k, v [T, KVH, D] (strided views of the qkv rows allowed). Every row must be a decode row, and
    slot_mapping[i] the slot of position seq_lens[i] - 1 (-1 where seq_lens[i] == 0), as every
    input builder produces; a row with any other in-range slot is not written and its output row
    is NaN (its write would race with other workgroups' reads), so such rows need kv_write and
    paged_attention instead. split_map: decode_split_map()'s result for this step (same meta,
    decode_version and partition) or None; the output is the same either way."""
    T, H, D = q.shape
    out = torch.empty(T, H * D, dtype=q.dtype, device=q.device)
    if T == 0:
        return out
    _check_gpu(q, k, v, k_cache, v_cache)
    NB, KVH, cd = _check_cache(k_cache, v_cache)
    _require(cd == D and q.stride(2) == 1 and q.dtype == torch.float16,
             "decode_kv_write_attention: q must be fp16 [T, H, D] with unit stride over D")
    _require(k.shape == (T, KVH, D) and v.shape == k.shape, "decode_kv_write_attention: k, v shape")
    _require(k.dtype == torch.float16 and v.dtype == torch.float16 and k.stride(2) == 1
             and v.stride(2) == 1, "decode_kv_write_attention: k, v must be fp16 rows")
    _require(decode_version in N.DECODE_VERSIONS, f"unknown decode version {decode_version!r}")
    S = meta.num_decode
    _require(S == T and meta.seq_lens.shape[0] == S,
             "decode_kv_write_attention: every row must be a decode row")
    bt, sl = _i32(meta.block_tables), _i32(meta.seq_lens)
    sm = meta.slot_mapping
    slots = sm if (sm.dtype == torch.int64 and sm.is_contiguous()) else sm.to(torch.int64).contiguous()
    _require(slots.shape[0] >= T, "decode_kv_write_attention: slot_mapping shorter than q")
    code, part = _decode_plan(S, int(meta.max_seq_len), decode_version, partition)
    ws_bytes = N.lib().ts_decode_workspace_bytes(code, S, H, KVH, D, int(meta.max_seq_len), part,
                                                 N.cu_count(q.device.index or 0))
    ws = _workspace(ws_bytes, q.device)
    N.check(N.lib().ts_decode_attention_kv_write(
        code, _ptr(q), q.stride(0), q.stride(1), _ptr(k), _ptr(v), k.stride(0), k.stride(1),
        v.stride(0), v.stride(1), _ptr(slots), _ptr(out), out.stride(0), _ptr(k_cache),
        _ptr(v_cache), NB, _ptr(bt), bt.stride(0), bt.shape[1], _ptr(sl), S, H, KVH, D,
        float(scale), int(meta.max_seq_len), int(part), _ptr(ws), ws_bytes, _stream(q),
        *_map_args(split_map)), "decode_kv_write_attention")
    return out


def decode_rope_kv_write_attention(qkv: torch.Tensor, positions: torch.Tensor,
                                   cos: torch.Tensor, sin: torch.Tensor, H: int, KVH: int, D: int,
                                   k_cache: torch.Tensor, v_cache: torch.Tensor, meta,
                                   scale: float, decode_version: str | None = None,
                                   partition: int | None = None,
                                   split_map=None) -> torch.Tensor | None:
    """The attention half of a pure-decode layer step in one launch: rope_(qkv, ...), kv_write
    of its k and v heads and paged_attention over the rotated q (model/qwen2.py:26-28, :89 with
    ops/triton_ops.py:60-71); returns the same [T, H*D] and leaves the same caches. qkv is left
    unrotated when the launch is fused (rotated in place when the library runs the rotation as its
    own launch), so only the returned output and the caches are defined afterwards. Returns None,
    having done nothing, when qkv's layout does not allow it (rows not 16-byte aligned): the
    caller then makes the separate calls. Every row must be a decode row, with slot_mapping and
    split_map as for decode_kv_write_attention."""
    T = qkv.shape[0]
    if not (qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.stride(0) % 8 == 0 and
            qkv.data_ptr() % 16 == 0 and k_cache.is_contiguous() and v_cache.is_contiguous()):
        return None
    out = torch.empty(T, H * D, dtype=qkv.dtype, device=qkv.device)
    if T == 0:
        return out
    _check_gpu(qkv, positions, cos, sin, k_cache, v_cache)
    NB, ckvh, cd = _check_cache(k_cache, v_cache)
    _require(qkv.dtype == torch.float16 and qkv.shape[1] >= (H + 2 * KVH) * D,
             "decode_rope_kv_write_attention: qkv must be fp16 [T, (H + 2 KVH) D]")
    _require(ckvh == KVH and cd == D, "decode_rope_kv_write_attention: cache shape mismatch")
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32 and cos.is_contiguous()
             and sin.is_contiguous() and cos.shape == sin.shape and cos.shape[-1] == D // 2,
             "decode_rope_kv_write_attention: tables must be contiguous fp32 [max_len, D / 2]")
    _require(decode_version in N.DECODE_VERSIONS, f"unknown decode version {decode_version!r}")
    S = meta.num_decode
    _require(S == T and meta.seq_lens.shape[0] == S,
             "decode_rope_kv_write_attention: every row must be a decode row")
    bt, sl = _i32(meta.block_tables), _i32(meta.seq_lens)
    pos = positions if (positions.dtype == torch.int64 and positions.is_contiguous()) \
        else positions.to(torch.int64).contiguous()
    sm = meta.slot_mapping
    slots = sm if (sm.dtype == torch.int64 and sm.is_contiguous()) else sm.to(torch.int64).contiguous()
    _require(slots.shape[0] >= T and pos.shape[0] >= T,
             "decode_rope_kv_write_attention: slot_mapping / positions shorter than qkv")
    code, part = _decode_plan(S, int(meta.max_seq_len), decode_version, partition)
    ws_bytes = N.lib().ts_decode_workspace_bytes(code, S, H, KVH, D, int(meta.max_seq_len), part,
                                                 N.cu_count(qkv.device.index or 0))
    ws = _workspace(ws_bytes, qkv.device)
    N.check(N.lib().ts_decode_rope_kv_write_attention(
        code, _ptr(qkv), qkv.stride(0), _ptr(pos), _ptr(cos), _ptr(sin), cos.shape[0], _ptr(out),
        out.stride(0), _ptr(k_cache), _ptr(v_cache), NB, _ptr(slots), _ptr(bt), bt.stride(0),
        bt.shape[1], _ptr(sl), S, H, KVH, D, float(scale), int(meta.max_seq_len), int(part),
        _ptr(ws), ws_bytes, _stream(qkv), *_map_args(split_map)), "decode_rope_kv_write_attention")
    return out


# ------------------------------------------------------------------------------------------
# W8A16 (ops/triton_w8a16.py:38-51, ops/triton_ops.py:74-91)
# ------------------------------------------------------------------------------------------
def w8a16_linear(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor,
                 bias: torch.Tensor | None, cfg=None) -> torch.Tensor:
    """y = x . (wq * scale)^T + bias, x fp16 [M, K], wq int8 [N, K], scale fp32 or fp16 [N].
    cfg = (variant, splits) of ts_w8a16_gemm_v (the reference passes its tuned Triton config in
    this position, ops/triton_ops.py:80-86); None takes the active variant table's choice for
    (N, K, M's bucket), or the library's own plan."""
    x = x.contiguous()
    M, K = x.shape
    Nn, Kw = wq.shape
    _require(Kw == K, f"w8a16: x has K={K}, weight has K={Kw}")
    _require(x.dtype == torch.float16, "w8a16: activations must be fp16")
    _require(wq.dtype == torch.int8 and wq.is_contiguous(), "w8a16: weight must be int8 row-major")
    _require(scale.dtype in (torch.float32, torch.float16) and scale.numel() == Nn,
             "w8a16: scale must be fp32 or fp16 [N]")
    y = torch.empty(M, Nn, dtype=x.dtype, device=x.device)
    if M == 0:
        return y
    _check_gpu(x, wq, scale)
    sc = scale.contiguous()
    b = None
    if bias is not None:
        _require(bias.numel() == Nn, "w8a16: bias must be [N]")
        b = bias.to(torch.float16).contiguous()
    cus = N.cu_count(x.device.index or 0)
    variant, splits = tuner.w8a16_choice(Nn, K, M) if cfg is None else (int(cfg[0]), int(cfg[1]))
    if variant == 0 and splits == 0:
        ws_bytes = N.lib().ts_w8a16_workspace_bytes(M, Nn, K, cus)
        ws = _workspace(ws_bytes, x.device)
        N.check(N.lib().ts_w8a16_gemm(_ptr(x), x.stride(0), _ptr(wq), _ptr(sc),
                                      1 if sc.dtype == torch.float16 else 0, _ptr(b), _ptr(y),
                                      y.stride(0), M, Nn, K, _ptr(ws), ws_bytes, _stream(x)),
                "w8a16_gemm")
        return y
    ws_bytes = N.lib().ts_w8a16_workspace_bytes_v(M, Nn, K, variant, splits, cus)
    ws = _workspace(ws_bytes, x.device)
    N.check(N.lib().ts_w8a16_gemm_v(_ptr(x), x.stride(0), _ptr(wq), _ptr(sc),
                                    1 if sc.dtype == torch.float16 else 0, _ptr(b), _ptr(y),
                                    y.stride(0), M, Nn, K, variant, splits, _ptr(ws), ws_bytes,
                                    _stream(x)), "w8a16_gemm_v")
    return y


def w8a16_glu(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor,
               bias: torch.Tensor | None = None, cfg=None) -> torch.Tensor:
    """silu(gate) * up of the fused gate_up W8A16 linear in one library call: wq int8 [2I, K] =
    [gate; up], out fp16 [M, I]. Equal, bit for bit, to silu_mul(w8a16_linear(x, wq, scale,
    bias, cfg)) (model/qwen2.py:35-36 with ops/triton_silu_mul.py:21-28): the product is planned
    for the [M, 2I] shape, so the same split and tile choice applies, and the [M, 2I]
    intermediate is never written. cfg as for w8a16_linear (the table entry of the gate_up
    shape)."""
    x = x.contiguous()
    M, K = x.shape
    Nn, Kw = wq.shape
    _require(Kw == K, f"w8a16_glu: x has K={K}, weight has K={Kw}")
    _require(Nn % 2 == 0, "w8a16_glu: weight must hold [gate; up] (an even number of rows)")
    _require(x.dtype == torch.float16, "w8a16_glu: activations must be fp16")
    _require(wq.dtype == torch.int8 and wq.is_contiguous(), "w8a16_glu: weight must be int8 row-major")
    _require(scale.dtype in (torch.float32, torch.float16) and scale.numel() == Nn,
             "w8a16_glu: scale must be fp32 or fp16 [2I]")
    inter = Nn // 2
    out = torch.empty(M, inter, dtype=x.dtype, device=x.device)
    if M == 0:
        return out
    _check_gpu(x, wq, scale)
    sc = scale.contiguous()
    b = None
    if bias is not None:
        _require(bias.numel() == Nn, "w8a16_glu: bias must be [2I]")
        b = bias.to(torch.float16).contiguous()
    cus = N.cu_count(x.device.index or 0)
    variant, splits = tuner.w8a16_choice(Nn, K, M) if cfg is None else (int(cfg[0]), int(cfg[1]))
    ws_bytes = N.lib().ts_w8a16_glu_workspace_bytes(M, inter, K, variant, splits, cus)
    ws = _workspace(ws_bytes, x.device)
    N.check(N.lib().ts_w8a16_glu(_ptr(x), x.stride(0), _ptr(wq), _ptr(sc),
                                 1 if sc.dtype == torch.float16 else 0, _ptr(b), _ptr(out),
                                 out.stride(0), M, inter, K, variant, splits, _ptr(ws), ws_bytes,
                                 _stream(x)), "w8a16_glu")
    return out


def w8a16_add_rmsnorm(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor,
                      bias: torch.Tensor | None, residual: torch.Tensor, w: torch.Tensor,
                      eps: float, cfg=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(out, new_residual) = rmsnorm_residual(w8a16_linear(x, wq, scale, bias, cfg), residual,
    w, eps), bit for bit, in two launches: the product, then the norm, which reduces the
    product's split-K partials itself when the plan splits K (no reduction launch of its own)."""
    x = x.contiguous()
    M, K = x.shape
    Nn, Kw = wq.shape
    _require(Kw == K, f"w8a16_add_rmsnorm: x has K={K}, weight has K={Kw}")
    _require(x.dtype == torch.float16, "w8a16_add_rmsnorm: activations must be fp16")
    _require(wq.dtype == torch.int8 and wq.is_contiguous(),
             "w8a16_add_rmsnorm: weight must be int8 row-major")
    _require(scale.dtype in (torch.float32, torch.float16) and scale.numel() == Nn,
             "w8a16_add_rmsnorm: scale must be fp32 or fp16 [N]")
    residual = _rows(residual, "w8a16_add_rmsnorm")
    _require(residual.shape == (M, Nn), "w8a16_add_rmsnorm: residual must be [M, N]")
    w = w.contiguous()
    _require(w.shape == (Nn,) and w.dtype == torch.float16, "w8a16_add_rmsnorm: norm weight must be fp16 [N]")
    out = torch.empty(M, Nn, dtype=x.dtype, device=x.device)
    res_out = torch.empty_like(out)
    if M == 0:
        return out, res_out
    _check_gpu(x, wq, scale, residual, w)
    sc = scale.contiguous()
    b = None
    if bias is not None:
        _require(bias.numel() == Nn, "w8a16_add_rmsnorm: bias must be [N]")
        b = bias.to(torch.float16).contiguous()
    cus = N.cu_count(x.device.index or 0)
    variant, splits = tuner.w8a16_choice(Nn, K, M) if cfg is None else (int(cfg[0]), int(cfg[1]))
    ws_bytes = N.lib().ts_w8a16_add_rmsnorm_workspace_bytes(M, Nn, K, variant, splits, cus)
    ws = _workspace(ws_bytes, x.device)
    N.check(N.lib().ts_w8a16_add_rmsnorm(
        _ptr(x), x.stride(0), _ptr(wq), _ptr(sc), 1 if sc.dtype == torch.float16 else 0, _ptr(b),
        _ptr(residual), residual.stride(0), _ptr(w), _ptr(out), out.stride(0), _ptr(res_out),
        res_out.stride(0), M, Nn, K, float(eps), variant, splits, _ptr(ws), ws_bytes,
        _stream(x)), "w8a16_add_rmsnorm")
    return out, res_out


def linear_rmsnorm_residual(x: torch.Tensor, lw: LinearWeight, residual: torch.Tensor,
                            w: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """rmsnorm_residual(linear(x, lw), residual, w, eps) (model/qwen2.py:84-92, o_proj then
    post_attention_layernorm, down_proj then the next norm): one fused call for int8 weights,
    the two calls otherwise."""
    if not lw.quantized:
        return rmsnorm_residual(linear(x, lw), residual, w, eps)
    return w8a16_add_rmsnorm(x, lw.w, lw.scale, lw.b, residual, w, eps)


def gate_up_silu(x: torch.Tensor, lw: LinearWeight) -> torch.Tensor:
    """silu_mul(linear(x, gate_up)) (model/qwen2.py:36): one fused call for int8 weights, the
    two calls otherwise."""
    if not lw.quantized:
        return silu_mul(F.linear(x, lw.w, lw.b))
    return w8a16_glu(x, lw.w, lw.scale, lw.b)


def linear(x: torch.Tensor, lw: LinearWeight) -> torch.Tensor:
    """fp16 weights stay on the vendor BLAS (F.linear, as ops/triton_ops.py:75-76 keeps cuBLAS);
    int8 weights take the W8A16 kernel at every M (the library picks its small-M streaming or
    MFMA tile path), replacing the reference's dequantise + cuBLAS route for M > 256."""
    if not lw.quantized:
        return F.linear(x, lw.w, lw.b)
    return w8a16_linear(x, lw.w, lw.scale, lw.b)


def lm_head_int8(h: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """int8 tied lm head (ops/triton_ops.py:88-91)."""
    return w8a16_linear(h, wq, scale, None)


def logits_int8(hidden: torch.Tensor, sample_indices: torch.Tensor, wq: torch.Tensor,
                scale: torch.Tensor) -> torch.Tensor:
    """Logits of the sampling rows, [S, V] fp32, through the int8 tied lm head in one launch:
    equal to lm_head_int8(hidden[sample_indices], wq, scale).float() (model/qwen2.py:94-99)."""
    _check_gpu(hidden, sample_indices, wq, scale)
    _require(hidden.dim() == 2 and hidden.dtype == torch.float16, "logits_int8: hidden must be fp16 [T, H]")
    if not (hidden.stride(1) == 1 and hidden.stride(0) % 8 == 0 and hidden.data_ptr() % 16 == 0):
        hidden = hidden.contiguous()
    T, Hd = hidden.shape
    V, Kw = wq.shape
    _require(Kw == Hd, f"logits_int8: hidden has {Hd} features, weight has {Kw}")
    _require(wq.dtype == torch.int8 and wq.is_contiguous(), "logits_int8: weight must be int8 row-major")
    _require(scale.dtype in (torch.float32, torch.float16) and scale.numel() == V,
             "logits_int8: scale must be fp32 or fp16 [V]")
    idx = sample_indices.reshape(-1).to(torch.int64).contiguous()
    S = idx.numel()
    out = torch.empty(S, V, dtype=torch.float32, device=hidden.device)
    if S == 0:
        return out
    _require(T > 0, "logits_int8: no hidden rows to sample from")
    sc = scale.contiguous()
    cus = N.cu_count(hidden.device.index or 0)
    ws_bytes = N.lib().ts_logits_int8_workspace_bytes(S, V, Hd, cus)
    ws = _workspace(ws_bytes, hidden.device)
    N.check(N.lib().ts_logits_int8(_ptr(hidden), hidden.stride(0), T, _ptr(idx), S, _ptr(wq),
                                   _ptr(sc), 1 if sc.dtype == torch.float16 else 0, _ptr(out),
                                   out.stride(0), V, Hd, _ptr(ws), ws_bytes, _stream(hidden)),
            "logits_int8")
    return out


# ------------------------------------------------------------------------------------------
# fused small ops (ops/triton_rmsnorm.py:30-46, ops/triton_rope.py:27-31,
# ops/triton_silu_mul.py:21-28)
# ------------------------------------------------------------------------------------------
def _rows(x: torch.Tensor, what: str) -> torch.Tensor:
    _check_gpu(x)
    _require(x.dim() == 2 and x.dtype == torch.float16, f"{what}: expected fp16 [T, N]")
    return x if (x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0) \
        else x.contiguous()


def rmsnorm_residual(x: torch.Tensor, residual: torch.Tensor | None, w: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(out, new_residual) with new_residual = x + residual (fp16) or x itself when residual is
    None, out = rmsnorm(new_residual) (ops/triton_rmsnorm.py:30-46)."""
    x = _rows(x, "rmsnorm")
    T, Nf = x.shape
    out = torch.empty(T, Nf, dtype=x.dtype, device=x.device)
    w = w.contiguous()
    _require(w.shape == (Nf,) and w.dtype == torch.float16, "rmsnorm: weight must be fp16 [N]")
    if residual is None:
        N.check(N.lib().ts_rmsnorm(_ptr(x), x.stride(0), None, 0, _ptr(w), _ptr(out), out.stride(0),
                                   None, 0, T, Nf, float(eps), _stream(x)), "rmsnorm")
        return out, x
    residual = _rows(residual, "rmsnorm")
    _require(residual.shape == x.shape, "rmsnorm: residual shape differs from x")
    res_out = torch.empty_like(out)
    N.check(N.lib().ts_rmsnorm(_ptr(x), x.stride(0), _ptr(residual), residual.stride(0), _ptr(w),
                               _ptr(out), out.stride(0), _ptr(res_out), res_out.stride(0), T, Nf,
                               float(eps), _stream(x)), "rmsnorm")
    return out, res_out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return rmsnorm_residual(x, None, w, eps)[0]


def rope_(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
          H: int, KVH: int, D: int) -> None:
    """In-place rotate-half RoPE on the q and k heads of qkv [T, (H + 2 KVH) D]; cos / sin are
    the fp32 tables [max_len, D / 2] (ops/triton_rope.py:27-31)."""
    _check_gpu(qkv, positions, cos, sin)
    T = qkv.shape[0]
    _require(qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.dtype == torch.float16,
             "rope: qkv must be fp16 rows with unit stride")
    _require(qkv.shape[1] >= (H + KVH) * D, "rope: qkv is narrower than the q and k heads")
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32 and cos.is_contiguous()
             and sin.is_contiguous() and cos.shape == sin.shape and cos.shape[-1] == D // 2,
             "rope: tables must be contiguous fp32 [max_len, D / 2]")
    pos = positions if (positions.dtype == torch.int64 and positions.is_contiguous()) \
        else positions.to(torch.int64).contiguous()
    N.check(N.lib().ts_rope(_ptr(qkv), qkv.stride(0), _ptr(pos), _ptr(cos), _ptr(sin),
                            cos.shape[0], T, H, KVH, D, _stream(qkv)), "rope")


def rope_kv_write_(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                   sin: torch.Tensor, H: int, KVH: int, D: int, k_cache: torch.Tensor,
                   v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> bool:
    """rope_(qkv, ...) then kv_write(k, v, k_cache, v_cache, slot_mapping) of qkv's k and v
    heads, in one pass over each token row (ops/triton_rope.py:27-31 then
    ops/triton_kv_write.py:28-35); the same bits as the two calls. Returns False, having done
    nothing, when qkv's layout does not allow the fused pass (rows not 16-byte aligned): the
    caller then makes the two calls."""
    _check_gpu(qkv, positions, cos, sin, k_cache, v_cache, slot_mapping)
    T = qkv.shape[0]
    if not (qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.stride(0) % 8 == 0 and
            qkv.data_ptr() % 16 == 0 and k_cache.is_contiguous() and v_cache.is_contiguous()):
        return False
    _require(qkv.dtype == torch.float16 and qkv.shape[1] >= (H + 2 * KVH) * D,
             "rope_kv_write: qkv must be fp16 [T, (H + 2 KVH) D]")
    NB, ckvh, cd = _check_cache(k_cache, v_cache)
    _require(ckvh == KVH and cd == D, "rope_kv_write: cache shape mismatch")
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32 and cos.is_contiguous()
             and sin.is_contiguous() and cos.shape == sin.shape and cos.shape[-1] == D // 2,
             "rope_kv_write: tables must be contiguous fp32 [max_len, D / 2]")
    _require(slot_mapping.shape[0] >= T, "rope_kv_write: slot_mapping shorter than qkv")
    pos = positions if (positions.dtype == torch.int64 and positions.is_contiguous()) \
        else positions.to(torch.int64).contiguous()
    slots = slot_mapping if (slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous()) \
        else slot_mapping.to(torch.int64).contiguous()
    N.check(N.lib().ts_rope_kv_write(_ptr(qkv), qkv.stride(0), _ptr(pos), _ptr(cos), _ptr(sin),
                                     cos.shape[0], T, H, KVH, D, _ptr(k_cache), _ptr(v_cache),
                                     NB, _ptr(slots), _stream(qkv)), "rope_kv_write")
    return True


def linear_rope_kv_write(x: torch.Tensor, lw: LinearWeight, positions: torch.Tensor,
                         cos: torch.Tensor, sin: torch.Tensor, H: int, KVH: int, D: int,
                         k_cache: torch.Tensor, v_cache: torch.Tensor,
                         slot_mapping: torch.Tensor) -> torch.Tensor:
    """qkv = linear(x, lw), then rope_kv_write_(qkv, ...) (model/qwen2.py:26-28, :89); returns
    qkv with q and k rotated, the rotated k and the v rows in the caches, the same bits as the
    calls it replaces. For int8 weights one call (ts_w8a16_qkv_rope_kv_write: the rotation and
    the cache rows in the product's epilogue where the plan allows, else its two launches)."""
    if not lw.quantized:
        qkv = linear(x, lw)
        if not rope_kv_write_(qkv, positions, cos, sin, H, KVH, D, k_cache, v_cache, slot_mapping):
            rope_(qkv, positions, cos, sin, H, KVH, D)
            T = qkv.shape[0]
            kv_write(qkv[:, H * D:(H + KVH) * D].view(T, KVH, D), qkv[:, (H + KVH) * D:].view(T, KVH, D),
                     k_cache, v_cache, slot_mapping)
        return qkv
    x = x.contiguous()
    M, K = x.shape
    wq, scale = lw.w, lw.scale
    Nn = (H + 2 * KVH) * D
    _require(x.dtype == torch.float16 and wq.dtype == torch.int8 and wq.is_contiguous() and
             tuple(wq.shape) == (Nn, K), "linear_rope_kv_write: int8 [(H + 2 KVH) D, K] weight")
    _require(scale.dtype in (torch.float32, torch.float16) and scale.numel() == Nn,
             "linear_rope_kv_write: scale must be fp32 or fp16 [N]")
    qkv = torch.empty(M, Nn, dtype=x.dtype, device=x.device)
    if M == 0:
        return qkv
    _check_gpu(x, wq, scale, positions, cos, sin, k_cache, v_cache, slot_mapping)
    NB, ckvh, cd = _check_cache(k_cache, v_cache)
    _require(ckvh == KVH and cd == D, "linear_rope_kv_write: cache shape mismatch")
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32 and cos.is_contiguous()
             and sin.is_contiguous() and cos.shape == sin.shape and cos.shape[-1] == D // 2,
             "linear_rope_kv_write: tables must be contiguous fp32 [max_len, D / 2]")
    _require(slot_mapping.shape[0] >= M and positions.shape[0] >= M,
             "linear_rope_kv_write: slot_mapping / positions shorter than x")
    pos = positions if (positions.dtype == torch.int64 and positions.is_contiguous()) \
        else positions.to(torch.int64).contiguous()
    slots = slot_mapping if (slot_mapping.dtype == torch.int64 and slot_mapping.is_contiguous()) \
        else slot_mapping.to(torch.int64).contiguous()
    sc = scale.contiguous()
    b = None if lw.b is None else lw.b.to(torch.float16).contiguous()
    cus = N.cu_count(x.device.index or 0)
    variant, splits = tuner.w8a16_choice(Nn, K, M)
    ws_bytes = N.lib().ts_w8a16_workspace_bytes_v(M, Nn, K, variant, splits, cus)
    ws = _workspace(ws_bytes, x.device)
    N.check(N.lib().ts_w8a16_qkv_rope_kv_write(
        _ptr(x), x.stride(0), _ptr(wq), _ptr(sc), 1 if sc.dtype == torch.float16 else 0, _ptr(b),
        _ptr(qkv), qkv.stride(0), M, K, H, KVH, D, _ptr(pos), _ptr(cos), _ptr(sin), cos.shape[0],
        _ptr(k_cache), _ptr(v_cache), NB, _ptr(slots), variant, splits, _ptr(ws), ws_bytes,
        _stream(x)), "w8a16_qkv_rope_kv_write")
    return qkv


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for gu = [gate | up] rows (ops/triton_silu_mul.py:21-28)."""
    gu = _rows(gu, "silu_mul")
    T, two_i = gu.shape
    inter = two_i // 2
    out = torch.empty(T, inter, dtype=gu.dtype, device=gu.device)
    N.check(N.lib().ts_silu_mul(_ptr(gu), gu.stride(0), _ptr(out), out.stride(0), T, inter,
                                _stream(gu)), "silu_mul")
    return out
