"""TuringServe's per-step hot path on MI355X (gfx950): kv_write, paged decode and chunked-prefill
attention and the W8A16 GEMM as hand-written HIP kernels behind a C ABI, with a Python host that
keeps the reference's op signatures (``get_ops("reference" | "hip")``)."""

__version__ = "0.1.0"


def get_ops(kernels: str):
    from turingserve_amd.ops import get_ops as _get

    return _get(kernels)
