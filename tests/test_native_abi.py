"""The C-ABI library on the CPU: it loads, exports every entry point include/turingserve_hip.h
declares, and its host-side argument checks and size functions answer without touching a GPU."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from turingserve_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "turingserve_hip.h")
PROBES_HEADER = os.path.join(ROOT, "include", "turingserve_probes.h")


def declared_functions(header: str = HEADER) -> list[str]:
    text = open(header, encoding="utf-8").read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ts_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 10
    lib = N.lib()
    for name in names:
        assert hasattr(lib, name), f"{name} declared but not exported"
        assert name in N.SIGNATURES, f"{name} has no ctypes signature"
    assert set(N.SIGNATURES) == set(names)


def test_probes_are_a_separate_measurement_library():
    """The measurement probes are not part of the product ABI: declared in their own header,
    exported by libturingserve_probes.so only."""
    names = declared_functions(PROBES_HEADER)
    assert sorted(names) == ["ts_probe_gather", "ts_probe_gather_k_operand",
                             "ts_probe_gather_persistent", "ts_probe_mfma"]
    assert not set(names) & set(declared_functions())
    for name in names:
        assert not hasattr(N.lib(), name), f"{name} exported by the product library"
        assert hasattr(N.probes_lib(), name)
    assert set(N.PROBE_SIGNATURES) == set(names)
    st = N.probes_lib().ts_probe_mfma(0, 1, None, None)
    assert st == N.TS_ERR_INVALID_ARG and N.last_error() != ""
    # a persistent grid too small for the chunk list is refused before any launch
    buf = ctypes.c_uint32()
    st = N.probes_lib().ts_probe_gather_persistent(ctypes.addressof(buf), ctypes.addressof(buf),
                                                   100000, 4096, 1, 8, 0, ctypes.addressof(buf),
                                                   None)
    assert st == N.TS_ERR_INVALID_ARG and "more workgroups" in N.last_error()


def test_version_and_empty_error():
    assert N.version().startswith("turingserve_hip") and "gfx950" in N.version()


def test_invalid_arguments_return_status_and_message():
    lib = N.lib()
    st = lib.ts_kv_write(None, None, 0, 0, 0, 0, None, None, 1, None, 4, 2, 64, None)
    assert st == N.TS_ERR_INVALID_ARG and "null pointer" in N.last_error()
    st = lib.ts_decode_attention(9, None, 0, 0, None, 0, None, None, 1, None, 1, 1, None, 1, 2, 1,
                                 64, 1.0, 16, 0, None, 0, None, None, 0)
    assert st == N.TS_ERR_INVALID_ARG and "unknown version" in N.last_error()
    p = ctypes.c_void_p(256)            # never dereferenced: the call fails validation first
    st = lib.ts_decode_attention(2, p, 96, 96, p, 96, p, p, 4, p, 1, 1, p, 1, 2, 1, 96, 1.0,
                                 16, 0, None, 0, None, None, 0)
    assert st == N.TS_ERR_UNSUPPORTED and "head_dim 96" in N.last_error()
    st = lib.ts_w8a16_gemm(p, 12, p, p, 0, None, p, 8, 3, 8, 12, None, 0, None)
    assert st == N.TS_ERR_UNSUPPORTED and "multiple of 8" in N.last_error()
    with pytest.raises(ValueError, match="multiple of 8"):
        N.check(st, "w8a16")


def test_small_op_argument_checks():
    lib = N.lib()
    p = ctypes.c_void_p(256)            # never dereferenced: the call fails validation first
    assert lib.ts_rmsnorm(p, 1536, None, 0, p, p, 1536, None, 0, 4, 12, 1e-6, None) == \
        N.TS_ERR_UNSUPPORTED and "multiple of 8" in N.last_error()
    assert lib.ts_rmsnorm(None, 0, None, 0, None, None, 0, None, 0, 4, 64, 1e-6, None) == \
        N.TS_ERR_INVALID_ARG
    assert lib.ts_rope(p, 2048, p, p, p, 16, 4, 12, 2, 12, None) == N.TS_ERR_UNSUPPORTED
    assert lib.ts_silu_mul(p, 100, p, 50, 2, 50, None) == N.TS_ERR_UNSUPPORTED
    assert lib.ts_rmsnorm(None, 0, None, 0, None, None, 0, None, 0, 0, 64, 1e-6, None) == N.TS_OK
    assert lib.ts_rope(None, 0, None, None, None, 0, 0, 12, 2, 128, None) == N.TS_OK
    assert lib.ts_silu_mul(None, 0, None, 0, 0, 64, None) == N.TS_OK


def test_logits_argument_checks():
    lib = N.lib()
    p = ctypes.c_void_p(256)            # never dereferenced: the call fails validation first
    # hidden_size not a multiple of 8; null pointers; misaligned logits rows; no samples: no-op
    assert lib.ts_logits_int8(p, 1540, 4, p, 2, p, p, 0, p, 1000, 1000, 1540, None, 0, None) == \
        N.TS_ERR_UNSUPPORTED and "multiple of 8" in N.last_error()
    assert lib.ts_logits_int8(None, 1536, 4, None, 2, None, None, 0, None, 1000, 1000, 1536, None,
                              0, None) == N.TS_ERR_INVALID_ARG
    assert lib.ts_logits_int8(p, 1536, 4, p, 2, p, p, 0, p, 1002, 1001, 1536, None, 0, None) == \
        N.TS_ERR_INVALID_ARG and "logits rows" in N.last_error()
    assert lib.ts_logits_int8(None, 0, 0, None, 0, None, None, 0, None, 0, 1000, 1536, None, 0,
                              None) == N.TS_OK
    # the gathered product is planned exactly like the GEMM on those rows
    for S in (1, 49, 300):
        assert lib.ts_logits_int8_workspace_bytes(S, 151936, 1536, 256) == \
            lib.ts_w8a16_workspace_bytes(S, 151936, 1536, 256)


def test_add_rmsnorm_argument_checks_and_workspace():
    lib = N.lib()
    p = ctypes.c_void_p(256)            # never dereferenced: the call fails validation first
    eps = ctypes.c_float(1e-6)
    assert lib.ts_w8a16_add_rmsnorm(p, 1536, p, p, 0, None, p, 1536, p, p, 1536, p, 1536, 4,
                                    1540, 1536, eps, 0, 0, p, 1 << 20, None) == \
        N.TS_ERR_UNSUPPORTED and "multiple of 8" in N.last_error()
    assert lib.ts_w8a16_add_rmsnorm(p, 1536, p, p, 0, None, p, 1536, p, p, 1536, p, 1536, 4,
                                    16384, 1536, eps, 0, 0, p, 1 << 20, None) == \
        N.TS_ERR_UNSUPPORTED and "8192" in N.last_error()
    assert lib.ts_w8a16_add_rmsnorm(p, 1536, p, p, 0, None, None, 1536, p, p, 1536, p, 1536, 4,
                                    1536, 1536, eps, 0, 0, p, 1 << 20, None) == N.TS_ERR_INVALID_ARG
    assert lib.ts_w8a16_add_rmsnorm(None, 0, None, None, 0, None, None, 0, None, None, 0, None, 0,
                                    0, 1536, 1536, eps, 0, 0, None, 0, None) == N.TS_OK
    assert lib.ts_w8a16_add_rmsnorm(p, 1536, p, p, 0, None, p, 1536, p, p, 1536, p, 1536, 64,
                                    1536, 1536, eps, 1, 0, p, 1 << 20, None) == N.TS_ERR_UNSUPPORTED
    # split K: the partials (as ts_w8a16_gemm_v's); else the fp16 product rows for the norm
    for M, v, s in ((64, 0, 0), (64, 4, 8), (560, 0, 0), (9, 2, 4), (4, 1, 3)):
        ws = lib.ts_w8a16_add_rmsnorm_workspace_bytes(M, 1536, 8960, v, s, 256)
        part = lib.ts_w8a16_workspace_bytes_v(M, 1536, 8960, v, s, 256)
        assert ws == (part if part > 0 else M * 1536 * 2)
    assert lib.ts_w8a16_add_rmsnorm_workspace_bytes(1, 1536, 1536, 5, 0, 256) == 1536 * 2
    assert lib.ts_w8a16_add_rmsnorm_workspace_bytes(64, 1536, 1536, 1, 0, 256) == 0


def test_glu_argument_checks_and_workspace():
    lib = N.lib()
    p = ctypes.c_void_p(256)            # never dereferenced: the call fails validation first
    assert lib.ts_w8a16_glu(p, 1540, p, p, 0, None, p, 8960, 4, 8960, 1540, 0, 0, None, 0,
                            None) == N.TS_ERR_UNSUPPORTED and "multiple of 8" in N.last_error()
    assert lib.ts_w8a16_glu(p, 1536, p, p, 0, None, p, 8962, 4, 8960, 1536, 0, 0, None, 0,
                            None) == N.TS_ERR_INVALID_ARG and "out rows" in N.last_error()
    assert lib.ts_w8a16_glu(p, 1536, p, p, 0, None, p, 8960, 64, 8960, 1536, 1, 0, None, 0,
                            None) == N.TS_ERR_UNSUPPORTED                # streaming is M <= 32
    assert lib.ts_w8a16_glu(None, 0, None, None, 0, None, None, 0, 0, 8960, 1536, 0, 0, None, 0,
                            None) == N.TS_OK
    # planned as the [M, 2I] product: the same split-K partials as ts_w8a16_gemm_v's
    for M, v, s in ((560, 0, 0), (2048, 0, 0), (64, 2, 3), (200, 3, 1), (4, 1, 1), (4, 1, 3)):
        assert lib.ts_w8a16_glu_workspace_bytes(M, 8960, 1536, v, s, 256) == \
            lib.ts_w8a16_workspace_bytes_v(M, 17920, 1536, v, s, 256)
    assert lib.ts_w8a16_glu_workspace_bytes(1, 8960, 1536, 1, 0, 256) == \
        lib.ts_w8a16_workspace_bytes_v(1, 17920, 1536, 1, 0, 256) > 0
    assert lib.ts_w8a16_glu_workspace_bytes(4, 8960, 1536, 1, 1, 256) == 0
    # M <= 16 (and the skinny variant up to M = 64) takes the skinny kernel, whole K per
    # workgroup: no split-K workspace
    for M in (1, 7, 16):
        assert lib.ts_w8a16_glu_workspace_bytes(M, 8960, 1536, 0, 0, 256) == 0
    # ... except long-K products whose 16-row tiles would cover under half the CUs (the down
    # projection: 96 of them), which take 128 x 32 tiles split 16 ways over K from M = 5 (the
    # VALU kernel, no workspace, below), and 8 ways at M = 64 (two 32-row tiles), about three
    # workgroups per four CUs
    for M in (1, 4):
        assert lib.ts_w8a16_workspace_bytes(M, 1536, 8960, 256) == 0
    for M in (5, 7, 16, 32):
        assert lib.ts_w8a16_workspace_bytes(M, 1536, 8960, 256) == 16 * M * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes(64, 1536, 8960, 256) == 8 * 64 * 1536 * 4
    # short-K products with many output channels (gate_up, 140 tiles of 128 rows) at M = 9 to
    # 32: 128 x 32 tiles, no split, no workspace; the skinny kernel below that
    for M in (9, 16, 32):
        assert lib.ts_w8a16_workspace_bytes(M, 17920, 1536, 256) == 0
    # the split 128 x 32 rule reaches M = 96 (three 32-row tiles, 4 splits of 6 K steps at
    # K = 1536, 6 splits at K = 8960); past it 128 x 64 tiles split while each split keeps 20 K
    # steps and the partials fit 8 MiB (7 splits of the down projection at M = 128 and 192)
    assert lib.ts_w8a16_workspace_bytes(96, 1536, 1536, 256) == 4 * 96 * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes(96, 2048, 1536, 256) == 4 * 96 * 2048 * 4
    assert lib.ts_w8a16_workspace_bytes(96, 1536, 8960, 256) == 6 * 96 * 1536 * 4
    for M in (128, 192):
        assert lib.ts_w8a16_workspace_bytes(M, 1536, 8960, 256) == 7 * M * 1536 * 4
    # ... and where the partial budget leaves them unsplit on under 2/3 of the CUs (long K,
    # M = 704 to 896 here), 128 x 128 tiles split 3 ways; past that, unsplit
    for M in (768, 896):
        assert lib.ts_w8a16_workspace_bytes(M, 1536, 8960, 256) == 3 * M * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes(1024, 1536, 8960, 256) == 0
    for M in (1, 16, 33, 64):
        assert lib.ts_w8a16_glu_workspace_bytes(M, 8960, 1536, 5, 0, 256) == 0
        assert lib.ts_w8a16_workspace_bytes_v(M, 2048, 1536, 5, 0, 256) == 0
    assert lib.ts_w8a16_workspace_bytes(64, 1536, 8960, 256) > 0     # wide 128 x 32, split K
    assert lib.ts_w8a16_glu(p, 1536, p, p, 0, None, p, 8960, 65, 8960, 1536, 5, 0, None, 0,
                            None) == N.TS_ERR_UNSUPPORTED                # skinny is M <= 64
    # the VALU path (variant 7): M <= 4, one K split, no workspace
    for M in (1, 4):
        assert lib.ts_w8a16_workspace_bytes_v(M, 1536, 8960, 7, 0, 256) == 0
        assert lib.ts_w8a16_glu_workspace_bytes(M, 8960, 1536, 7, 1, 256) == 0
    assert lib.ts_w8a16_workspace_bytes_v(5, 1536, 8960, 7, 0, 256) == 0      # not available
    assert lib.ts_w8a16_glu(p, 1536, p, p, 0, None, p, 8960, 5, 8960, 1536, 7, 0, None, 0,
                            None) == N.TS_ERR_UNSUPPORTED                # VALU path is M <= 4
    assert lib.ts_w8a16_glu(p, 1536, p, p, 0, None, p, 8960, 2, 8960, 1536, 7, 2, None, 0,
                            None) == N.TS_ERR_UNSUPPORTED                # and never splits K


def test_zero_size_calls_are_no_ops():
    lib = N.lib()
    assert lib.ts_kv_write(None, None, 0, 0, 0, 0, None, None, 0, None, 0, 2, 64, None) == N.TS_OK
    assert lib.ts_decode_attention(0, None, 0, 0, None, 0, None, None, 0, None, 0, 0, None, 0, 12,
                                   2, 128, 1.0, 0, 0, None, 0, None, None, 0) == N.TS_OK
    assert lib.ts_w8a16_gemm(None, 0, None, None, 0, None, None, 0, 0, 16, 16, None, 0,
                             None) == N.TS_OK


def test_workspace_sizes():
    lib = N.lib()

    def v3_bytes(rows_per_seq, S=64, H=12, D=128):
        n = S * rows_per_seq * H                 # partial rows x heads: D fp32 (acc), 2 fp32
        a256 = lambda x: (x + 255) // 256 * 256
        return a256(n * D * 4) + 2 * a256(n * 4) + a256(S * 4)

    # fixed grid: 4096 / 256 = 16 split rows per sequence
    want = v3_bytes(16)
    assert lib.ts_decode_workspace_bytes(3, 64, 12, 2, 128, 4096, 256, 256) == want
    assert lib.ts_decode_workspace_bytes(2, 64, 12, 2, 128, 4096, 0, 256) == 0
    assert lib.ts_decode_workspace_bytes(1, 64, 12, 2, 128, 4096, 0, 256) == 0
    # own-length v3 (partition 0): ceil(max blocks / 24) split rows per sequence, at most 32
    assert lib.ts_decode_workspace_bytes(3, 64, 12, 2, 128, 4096, 0, 256) == v3_bytes(11)
    assert lib.ts_decode_workspace_bytes(3, 64, 12, 2, 128, 32768, 0, 256) == v3_bytes(32)
    # the automatic policy splits 64 x 2 (seq, KV head) workgroups < 512 resident ones, with the
    # fixed grid when a partition is named and the own-length schedule otherwise ...
    assert lib.ts_decode_workspace_bytes(0, 64, 12, 2, 128, 4096, 256, 256) == want
    assert lib.ts_decode_workspace_bytes(0, 64, 12, 2, 128, 1024, 0, 256) == v3_bytes(3)
    # ... but not contexts of at most two minimum splits or a batch that fills the device
    assert lib.ts_decode_workspace_bytes(0, 64, 12, 2, 128, 256, 0, 256) == 0
    assert lib.ts_decode_workspace_bytes(0, 256, 12, 2, 128, 4096, 0, 256) == 0
    # W8A16: 128 x 128 tiles that cover the device need no workspace
    assert lib.ts_w8a16_workspace_bytes(2048, 17920, 1536, 256) == 0
    assert lib.ts_w8a16_workspace_bytes(64, 17920, 1536, 256) == 0      # 140 tiles of 128 x 64
    # 108 tiles of 128 x 64 for the 1.5B down projection at M = 560: split K in two (70 K
    # steps each, partials 2 x 560 x 1536 fp32 within the 8 MB floor); a third split would not
    # fit and K = 1536 (24 steps) never splits
    assert lib.ts_w8a16_workspace_bytes(560, 1536, 8960, 256) == 2 * 560 * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes(560, 1536, 1536, 256) == 0
    # M <= 16 takes the VALU or the skinny kernel (whole K per workgroup): no workspace
    assert lib.ts_w8a16_workspace_bytes(1, 2048, 1536, 256) == 0
    assert lib.ts_w8a16_workspace_bytes(16, 2048, 1536, 256) == 0
    # weight streaming (variant 1) at M = 1: 32 workgroups, split into 6 (K / 256) partial rows
    assert lib.ts_w8a16_workspace_bytes_v(1, 2048, 1536, 1, 0, 256) == 6 * 2048 * 4
    ws = lib.ts_w8a16_workspace_bytes_v(1, 1536, 8960, 1, 0, 256)
    assert ws > 0 and ws % (1536 * 4) == 0


def test_split_map_sizes_and_checks():
    lib = N.lib()
    # one header of 8 ints, 32 ints per launch slot of the v3 plan and one arrival counter per
    # (sequence, KV head, head group): the own-length schedule launches ceil(max blocks / 24)
    # slots per sequence (11 at 4096 tokens, 3 at 1024), the fixed grid 16 slots per sequence at
    # 4096 / 256; 64 sequences x 2 KV heads x 1 head group of counters
    assert lib.ts_decode_split_map_bytes(3, 64, 12, 2, 128, 4096, 0, 256) == (8 + 64 * 11 * 32 + 128) * 4
    assert lib.ts_decode_split_map_bytes(3, 64, 12, 2, 128, 4096, 256, 256) == (8 + 64 * 16 * 32 + 128) * 4
    assert lib.ts_decode_split_map_bytes(0, 64, 12, 2, 128, 1024, 0, 256) == (8 + 64 * 3 * 32 + 128) * 4
    # no split, no map: v1 / v2, AUTO resolving to v2, more than 4096 sequences
    assert lib.ts_decode_split_map_bytes(2, 64, 12, 2, 128, 4096, 0, 256) == 0
    assert lib.ts_decode_split_map_bytes(1, 64, 12, 2, 128, 4096, 0, 256) == 0
    assert lib.ts_decode_split_map_bytes(0, 256, 12, 2, 128, 4096, 0, 256) == 0
    assert lib.ts_decode_split_map_bytes(3, 4097, 12, 2, 128, 4096, 256, 256) == 0
    assert lib.ts_decode_split_map(3, None, 1, 1, 1, None, 0, 12, 2, 128, 4096, 0, None, 0,
                                   None) == N.TS_OK                     # empty batch
    st = lib.ts_decode_split_map(3, None, 1, 1, 1, None, 4097, 12, 2, 128, 4096, 0, None, 0, None)
    assert st == N.TS_ERR_UNSUPPORTED and "4096" in N.last_error()
    st = lib.ts_decode_split_map(7, None, 1, 1, 1, None, 4, 12, 2, 128, 4096, 0, None, 0, None)
    assert st == N.TS_ERR_INVALID_ARG and "unknown version" in N.last_error()
    st = lib.ts_decode_split_map(3, None, 1, 1, 1, None, 4, 12, 2, 128, 4096, 0, None, 0, None)
    assert st == N.TS_ERR_INVALID_ARG and "null pointer" in N.last_error()


def test_qkv_rope_kv_write_argument_checks():
    lib = N.lib()
    p = ctypes.c_void_p(256)            # never dereferenced: the call fails validation first
    assert lib.ts_w8a16_qkv_rope_kv_write(None, 0, None, None, 0, None, None, 0, 0, 1536, 12, 2,
                                          128, p, p, p, 16, p, p, 4, p, 0, 0, None, 0,
                                          None) == N.TS_OK                  # no rows
    st = lib.ts_w8a16_qkv_rope_kv_write(p, 1536, p, p, 0, None, p, 2048, 4, 1536, 12, 2, 128,
                                        None, p, p, 16, p, p, 4, p, 0, 0, None, 0, None)
    assert st == N.TS_ERR_INVALID_ARG and "null pointer" in N.last_error()
    st = lib.ts_w8a16_qkv_rope_kv_write(p, 1536, p, p, 0, None, p, 2048, 4, 1536, 0, 2, 128,
                                        p, p, p, 16, p, p, 4, p, 0, 0, None, 0, None)
    assert st == N.TS_ERR_INVALID_ARG and "head counts" in N.last_error()


def test_python_wrappers_reject_cpu_tensors():
    from turingserve_amd import hip_ops as K

    kc = torch.zeros(4, 2, 16, 64, dtype=torch.float16)
    k = torch.zeros(3, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        K.kv_write(k, k, kc, kc.clone(), torch.zeros(3, dtype=torch.int64))


def test_get_ops_namespaces():
    from turingserve_amd import get_ops

    ref = get_ops("reference")
    hip = get_ops("hip")
    assert ref.name == "reference" and hip.name == "hip"
    assert get_ops("triton").name == "hip"
    for op in ("kv_write", "paged_attention", "linear", "rmsnorm", "rope_", "silu_mul"):
        assert callable(getattr(hip, op))
    assert hip.kv_write.__module__ == "turingserve_amd.hip_ops"
    assert ref.kv_write.__module__ == "turingserve_amd.reference_ops"
    with pytest.raises(ValueError):
        get_ops("cuda")
