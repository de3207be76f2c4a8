"""ctypes binding of libturingserve_hip.so (the C ABI declared in include/turingserve_hip.h).

There is no fallback: if the library is missing or cannot be loaded, every call raises
``NativeLibraryError``. torch is imported first so that the library binds to the HIP runtime
torch already loaded (both carry the soname libamdhip64.so.7), which makes torch's streams and
allocations valid inside the library.
"""

from __future__ import annotations

import ctypes
import functools
import os

import torch  # noqa: F401  (loads the HIP runtime before the library)

# TS_HIP_LIB selects another build of the same library (e.g. to compare kernel variants).
LIB_PATH = os.environ.get("TS_HIP_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "lib", "libturingserve_hip.so")

TS_OK = 0
TS_ERR_INVALID_ARG = -1
TS_ERR_UNSUPPORTED = -2
TS_ERR_WORKSPACE = -3
TS_ERR_LAUNCH = -4
TS_ERR_DEVICE = -5
TS_NOALLOC_SCRATCH_BYTES = 16 << 20    # static split scratch of ts_decode_attention_kv_write_noalloc

DECODE_VERSIONS = {None: 0, "auto": 0, "v1": 1, "v2": 2, "v3": 3}

_p, _i32, _i64, _f32, _sz = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float,
                             ctypes.c_size_t)

# name -> (restype, argtypes); the order follows include/turingserve_hip.h
SIGNATURES = {
    "ts_version": (ctypes.c_char_p, []),
    "ts_last_error": (ctypes.c_char_p, []),
    "ts_device_cu_count": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "ts_kv_write": (ctypes.c_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _i64, _i32,
                                   _i32, _p]),
    "ts_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "ts_decode_attention": (ctypes.c_int, [_i32, _p, _i64, _i64, _p, _i64, _p, _p, _i64, _p, _i64,
                                           _i32, _p, _i32, _i32, _i32, _i32, _f32, _i32, _i32,
                                           _p, _sz, _p, _p, _sz]),
    "ts_w8a16_qkv_rope_kv_write": (ctypes.c_int, [_p, _i64, _p, _p, _i32, _p, _p, _i64, _i32, _i32,
                                                  _i32, _i32, _i32, _p, _p, _p, _i64, _p, _p,
                                                  _i64, _p, _i32, _i32, _p, _sz, _p]),
    "ts_decode_split_map_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "ts_decode_split_map": (ctypes.c_int, [_i32, _p, _i64, _i32, _i64, _p, _i32, _i32, _i32, _i32,
                                           _i32, _i32, _p, _sz, _p]),
    "ts_decode_attention_kv_write": (ctypes.c_int, [_i32, _p, _i64, _i64, _p, _p, _i64, _i64,
                                                    _i64, _i64, _p, _p, _i64, _p, _p, _i64, _p,
                                                    _i64, _i32, _p, _i32, _i32, _i32, _i32, _f32,
                                                    _i32, _i32, _p, _sz, _p, _p, _sz]),
    "ts_decode_attention_kv_write_noalloc": (ctypes.c_int, [_i32, _p, _i64, _i64, _p, _p, _i64,
                                                            _i64, _i64, _i64, _p, _p, _i64, _p,
                                                            _p, _i64, _p, _i64, _i32, _p, _i32,
                                                            _i32, _i32, _i32, _f32, _i32, _i32,
                                                            _p]),
    "ts_decode_rope_kv_write_attention": (ctypes.c_int, [_i32, _p, _i64, _p, _p, _p, _i64, _p,
                                                         _i64, _p, _p, _i64, _p, _p, _i64, _i32,
                                                         _p, _i32, _i32, _i32, _i32, _f32, _i32,
                                                         _i32, _p, _sz, _p, _p, _sz]),
    "ts_prefill_attention": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _i64,
                                            _i32, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                                            _f32, _p]),
    "ts_prefill_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ts_prefill_attention_ws": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p,
                                               _i64, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                               _i32, _i32, _f32, _p, _sz, _p]),
    "ts_paged_attention_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                                  _i32, _i32, _i32]),
    "ts_paged_attention": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _i64,
                                          _i32, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                          _i32, _f32, _i32, _i32, _p, _sz, _p]),
    "ts_w8a16_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "ts_w8a16_gemm": (ctypes.c_int, [_p, _i64, _p, _p, _i32, _p, _p, _i64, _i32, _i32, _i32, _p,
                                     _sz, _p]),
    "ts_w8a16_workspace_bytes_v": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ts_w8a16_gemm_v": (ctypes.c_int, [_p, _i64, _p, _p, _i32, _p, _p, _i64, _i32, _i32, _i32,
                                       _i32, _i32, _p, _sz, _p]),
    "ts_w8a16_glu_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ts_w8a16_glu": (ctypes.c_int, [_p, _i64, _p, _p, _i32, _p, _p, _i64, _i32, _i32, _i32, _i32,
                                    _i32, _p, _sz, _p]),
    "ts_w8a16_add_rmsnorm_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ts_w8a16_add_rmsnorm": (ctypes.c_int, [_p, _i64, _p, _p, _i32, _p, _p, _i64, _p, _p, _i64,
                                            _p, _i64, _i32, _i32, _i32, _f32, _i32, _i32, _p, _sz,
                                            _p]),
    "ts_logits_int8_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "ts_step_metadata": (ctypes.c_int, [_p, _i32, _i64, _i64, _i32, _i32, _i64, _p, _p, _p, _p,
                                        _p, _p, _p, _p]),
    "ts_logits_int8": (ctypes.c_int, [_p, _i64, _i64, _p, _i32, _p, _p, _i32, _p, _i64, _i32,
                                      _i32, _p, _sz, _p]),
    "ts_rmsnorm": (ctypes.c_int, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i32, _f32,
                                  _p]),
    "ts_rope": (ctypes.c_int, [_p, _i64, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p]),
    "ts_rope_kv_write": (ctypes.c_int, [_p, _i64, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p,
                                        _p, _i64, _p, _p]),
    "ts_silu_mul": (ctypes.c_int, [_p, _i64, _p, _i64, _i64, _i32, _p]),
}

# The measurement-only probes library (include/turingserve_probes.h): not part of the product ABI.
PROBE_SIGNATURES = {
    "ts_probe_gather": (ctypes.c_int, [_p, _p, _i32, _i32, _p, _p]),
    "ts_probe_mfma": (ctypes.c_int, [_i32, _i32, _p, _p]),
    "ts_probe_gather_persistent": (ctypes.c_int, [_p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p]),
    "ts_probe_gather_k_operand": (ctypes.c_int, [_p, _p, _i32, _i32, _p, _p]),
}


class NativeLibraryError(RuntimeError):
    """The gfx950 kernel library is missing or failed to load."""


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryError(
            f"{LIB_PATH} not found: build it with `python -m turingserve_amd.csrc.build` "
            "(there is no CPU fallback for the hip backend)")
    try:
        L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    except OSError as e:
        raise NativeLibraryError(f"cannot load {LIB_PATH}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


@functools.lru_cache(maxsize=1)
def probes_lib() -> ctypes.CDLL:
    """libturingserve_probes.so (measurement only, bench.py's calibration); loads the product
    library first, whose status codes and ts_last_error it shares."""
    lib()
    path = os.path.join(os.path.dirname(LIB_PATH), "libturingserve_probes.so")
    if not os.path.exists(path):
        raise NativeLibraryError(f"{path} not found: build it with `python -m turingserve_amd.csrc.build`")
    L = ctypes.CDLL(path)
    for name, (res, args) in PROBE_SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def last_error() -> str:
    return lib().ts_last_error().decode()


def check(status: int, what: str) -> None:
    """Turn a C status into the Python exception the reference's callers expect."""
    if status == TS_OK:
        return
    msg = f"{what}: {last_error()} (status {status})"
    if status in (TS_ERR_INVALID_ARG, TS_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


@functools.lru_cache(maxsize=16)
def cu_count(device_index: int) -> int:
    """Compute units of a device (the reference's cached num_sms, ops/triton_ops.py:29-32)."""
    n = ctypes.c_int(0)
    check(lib().ts_device_cu_count(device_index, ctypes.byref(n)), "device_cu_count")
    return n.value


def version() -> str:
    return lib().ts_version().decode()
