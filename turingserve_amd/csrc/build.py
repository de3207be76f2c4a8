"""Build libturingserve_hip.so (gfx950 only) from the .hip sources next to this file.

    python -m turingserve_amd.csrc.build           # compile every source, link the libraries

Each source is compiled on its own (in parallel) into ``_build/`` and linked into
``turingserve_amd/lib/libturingserve_hip.so``; the measurement probes (probes.hip, declared in
include/turingserve_probes.h, not part of the product ABI) go into their own
``libturingserve_probes.so``, linked against the product library. Packed-FP32 instructions are
disabled for every kernel (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_DIR = os.path.join(PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libturingserve_hip.so")
PROBES_PATH = os.path.join(LIB_DIR, "libturingserve_probes.so")
BUILD_DIR = os.path.join(HERE, "_build")
SOURCES = ["capi.hip", "kv_write.hip", "decode.hip", "prefill.hip", "ragged.hip", "w8a16.hip",
           "small_ops.hip", "metadata.hip"]
PROBE_SOURCES = ["probes.hip"]
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-source flags. Attention kernels keep their MFMA accumulators in VGPRs (gfx90a+ allows
# either file): with the default AGPR form the register allocator copied whole O^T accumulator
# sets between AGPRs around the rarely taken softmax rescale branch; the VGPR form needs no
# copies at the same occupancy. The GEMM keeps the default AGPR form: its widest tile holds 128
# accumulator registers per lane, which then live in AGPRs beside ~200 VGPRs instead of
# spilling out of a 256-register VGPR file.
SOURCE_FLAGS = {
    "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "ragged.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), *extra, "-c",
           os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _link(path: str, objs: list[str], libs: list[str]) -> None:
    tmp = path + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *libs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, path)


def build(verbose: bool = False, extra: list[str] | None = None) -> str:
    """Compile every source, link the product library and the probes library; returns the
    product library's path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    extra = list(extra or [])
    if verbose:
        extra.append("-Rpass-analysis=kernel-resource-usage")
    srcs = SOURCES + PROBE_SOURCES
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = dict(zip(srcs, ex.map(lambda s: _compile(s, extra), srcs)))
    _link(LIB_PATH, [objs[s] for s in SOURCES], [])
    _link(PROBES_PATH, [objs[s] for s in PROBE_SOURCES],
          [f"-L{LIB_DIR}", "-lturingserve_hip", "-Wl,-rpath,$ORIGIN"])
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv[1:]))
