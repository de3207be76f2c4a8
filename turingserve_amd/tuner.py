"""Variant-selection table for the HIP kernels: the role of the reference's tuner and tuning cache
(autopilot/tuner.py:56-134, consulted by ops/triton_ops.py:44-86, loaded by autopilot/startup.py:
20-43), for this backend's variants instead of Triton configs.

Each kernel has candidate variants per shape bucket; tune() times every candidate with HIP events
over graph-captured calls and keeps the fastest; the winners are stored in a JSON file whose name
follows the GPU, CU count, model and library / torch versions. At run time the ops look their
bucket up and round up to the next measured bucket, as the reference's lookup does (for W8A16
only M rounds; N and K must match); a miss takes the library's own plan. tune() records the M
buckets below the engine's token budget and the budget itself.

    kernel "decode": key (S, L)    (decode rows, max_seq_len)       -> {"version": "v2" | "v3",
                                                                         "partition": 0 | 256 | ...}
    kernel "w8a16":  key (N, K, M) (out features, in features, rows) -> {"variant": 0..7,
                                                                         "splits": 0..}

W8A16 variants (ts_w8a16_gemm_v): 0 the library's plan, 1 weight streaming (M <= 32),
2 128 x 64 wide tiles, 3 128 x 128 wide tiles, 4 128 x 32 wide tiles (128 x 64 in the fused
gated-MLP product), 5 skinny (M <= 64: whole K per workgroup, no split-K), 6 128 x 192 wide
tiles, 7 weight rows streamed on the VALU (M <= 4); splits 0 = the variant's own rule. Decode:
v2 (one workgroup per sequence and KV head group) or v3 with partition 0 (own-length split) or a
fixed partition in tokens. Every variant computes the same result up to fp32 summation order.
"""

from __future__ import annotations

import bisect
import hashlib
import json
import os
import tempfile

W8A16_M_BUCKETS = (1, 8, 16, 32, 64, 128, 256, 512, 768, 1024, 2048, 4096)
DECODE_PARTITIONS = (0, 256, 512, 1024)
FORMAT = 2                       # version of the JSON layout below


class VariantTable:
    """Measured choices: for each kernel, records (key, choice) with an integer tuple key.

    JSON layout: {"format": 2, "meta": {...}, "records": [{"kernel": k, "key": [..],
    "choice": {..}}, ...]} (records sorted by kernel and key, so equal tables serialise equally).
    """

    def __init__(self, meta: dict | None = None) -> None:
        self.meta = dict(meta or {})
        self._by_kernel: dict[str, dict[tuple[int, ...], dict]] = {}

    def set(self, kernel: str, key, choice: dict) -> None:
        self._by_kernel.setdefault(kernel, {})[tuple(int(k) for k in key)] = dict(choice)

    def records(self, kernel: str) -> dict[tuple[int, ...], dict]:
        return dict(self._by_kernel.get(kernel, {}))

    def lookup(self, kernel: str, key) -> dict | None:
        """The choice recorded under the smallest key (in tuple order) that is >= `key` in every
        component, or None. A query of a bucket the table did not measure therefore takes the
        next larger measured bucket."""
        want = tuple(int(k) for k in key)
        fits = [k for k in self._by_kernel.get(kernel, {})
                if len(k) == len(want) and all(a >= b for a, b in zip(k, want))]
        return self._by_kernel[kernel][min(fits)] if fits else None

    def to_json(self) -> str:
        recs = [{"kernel": kern, "key": list(key), "choice": choice}
                for kern in sorted(self._by_kernel)
                for key, choice in sorted(self._by_kernel[kern].items())]
        return json.dumps({"format": FORMAT, "meta": self.meta, "records": recs}, indent=1,
                          sort_keys=True)

    @classmethod
    def from_json(cls, text: str) -> "VariantTable":
        doc = json.loads(text)
        if not isinstance(doc, dict) or doc.get("format") != FORMAT:
            raise ValueError("not a variant table of this format")
        table = cls(doc.get("meta", {}))
        for rec in doc["records"]:
            if not (isinstance(rec["key"], list) and isinstance(rec["choice"], dict)):
                raise ValueError("malformed record")
            table.set(str(rec["kernel"]), rec["key"], rec["choice"])
        return table


ACTIVE = VariantTable()          # consulted by hip_ops


def set_active(table: VariantTable) -> None:
    global ACTIVE
    ACTIVE = table


def w8a16_choice(N: int, K: int, M: int) -> tuple[int, int]:
    """(variant, splits) for a W8A16 product: N and K must match a record exactly, M takes the
    smallest recorded M >= M (bisected over that shape's M list); else the library's own plan
    (0, 0). A streaming choice (variant 1) recorded for a bucket whose range reaches past
    M = 32 cannot apply and also falls back."""
    shape = sorted((k[2], c) for k, c in ACTIVE.records("w8a16").items() if k[:2] == (N, K))
    i = bisect.bisect_left([m for m, _ in shape], M)
    if i == len(shape):
        return 0, 0
    c = shape[i][1]
    variant, splits = int(c["variant"]), int(c["splits"])
    if (variant == 1 and M > 32) or (variant == 5 and M > 64) or (variant == 7 and M > 4):
        return 0, 0
    return variant, splits


def decode_choice(S: int, max_seq_len: int) -> tuple[str | None, int | None]:
    """(version, partition) for S decode rows at this max_seq_len, or (None, None)."""
    c = ACTIVE.lookup("decode", (S, max_seq_len))
    if c is None:
        return None, None
    return c["version"], int(c["partition"])


def cache_file_name(gpu: str, cus: int, model: str, lib_version: str, torch_version: str) -> str:
    """A file name that changes whenever any of the fields does: a readable prefix (GPU, CU count,
    model, with path-unsafe characters dropped) and a hash of all five fields."""
    digest = hashlib.sha256("\x1f".join([gpu, str(cus), model, lib_version, torch_version])
                            .encode()).hexdigest()[:16]
    readable = "-".join("".join(ch for ch in f if ch.isalnum() or ch in "._") or "x"
                        for f in (gpu, f"cu{cus}", model))
    return f"{readable}-{digest}.json"


def load_table(directory: str, name: str) -> VariantTable | None:
    """The table stored under `name`, or None if it is missing or unreadable (then tune again)."""
    try:
        with open(os.path.join(os.path.expanduser(directory), name), encoding="utf-8") as f:
            return VariantTable.from_json(f.read())
    except (OSError, ValueError, KeyError, TypeError):
        return None


def store_table(directory: str, name: str, table: VariantTable) -> str:
    """Write the table under `name`; a reader never sees a partial file (written to a temporary
    file in the same directory, then renamed over the target)."""
    d = os.path.expanduser(directory)
    os.makedirs(d, exist_ok=True)
    fd, tmp = tempfile.mkstemp(dir=d, prefix=".variant-", suffix=".json")
    try:
        with os.fdopen(fd, "w", encoding="utf-8") as f:
            f.write(table.to_json())
        os.replace(tmp, os.path.join(d, name))
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise
    return os.path.join(d, name)


def _ladder(lo: int, hi: int) -> list[int]:
    """lo, 2 lo, 4 lo, ... below hi, then hi."""
    return [lo << i for i in range(max(0, (hi - 1) // lo).bit_length()) if lo << i < hi] + [hi]


# ---- the measuring part (needs a GPU) -------------------------------------------------------------
def time_call(torch, fn, inner: int = 10, reps: int = 5) -> float:
    """Mean milliseconds of fn() from a hipGraph of `inner` back-to-back calls, replayed `reps`
    times after a warm-up replay (HIP events on the capturing stream)."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(inner):
            fn()
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / (reps * inner)


def w8a16_candidates(M: int) -> list[tuple[int, int]]:
    cands = [(0, 0), (2, 0), (2, 1), (2, 2), (2, 4), (3, 0), (3, 2), (4, 0), (4, 2), (6, 0), (6, 2)]
    if M <= 32:
        cands += [(1, 0), (1, 1), (1, 2), (1, 4)]
    if M <= 64:
        cands += [(5, 0)]
    if M <= 4:
        cands += [(7, 0)]
    return cands


def tune_w8a16(torch, shapes, ms, device="cuda", table: VariantTable | None = None,
               timer=time_call, cold_bytes: int = 512 << 20) -> VariantTable:
    """Time every W8A16 candidate for each (N, K) in `shapes` at each M in `ms` (bucket
    values); keep the fastest (ties go to the earlier candidate, the library's plan first).
    The weights are timed cold, as a model step meets them: consecutive calls cycle through
    copies of the weight that together exceed `cold_bytes` (past the 256 MB Infinity Cache)."""
    import itertools

    from turingserve_amd import hip_ops as K_

    table = table or VariantTable()
    g = torch.Generator(device=device).manual_seed(0)
    for (N, K) in shapes:
        wq = torch.randint(-127, 128, (N, K), generator=g, device=device, dtype=torch.int8)
        copies = [wq] + [wq.clone() for _ in range(max(1, -(-cold_bytes // (N * K)) - 1))]
        sc = torch.rand(N, generator=g, device=device) / 127 + 1e-4
        for M in ms:
            x = torch.randn(M, K, generator=g, device=device).half()
            best = None
            for (v, s) in w8a16_candidates(M):
                it = itertools.cycle(copies)
                t = timer(torch, lambda v=v, s=s: K_.w8a16_linear(x, next(it), sc, None, cfg=(v, s)),
                          inner=len(copies), reps=2)
                if best is None or t < best[0]:
                    best = (t, v, s)
            table.set("w8a16", (N, K, M), {"variant": best[1], "splits": best[2],
                                           "us": round(best[0] * 1e3, 2)})
    return table


def tune_decode(torch, H: int, KVH: int, D: int, seqs, lens, device="cuda",
                table: VariantTable | None = None, timer=time_call) -> VariantTable:
    """Time v2 and v3 (own-length and fixed partitions) for S decode rows of length L each."""
    from turingserve_amd import hip_ops as K_
    from turingserve_amd.metadata import AttentionMetadata

    table = table or VariantTable()
    g = torch.Generator(device=device).manual_seed(0)
    max_L = max(lens)
    nb_total = max(seqs) * (-(-max_L // 16)) + 8
    kc = torch.randn(nb_total, KVH, 16, D, generator=g, device=device).half()
    vc = torch.randn(nb_total, KVH, 16, D, generator=g, device=device).half()
    for S in seqs:
        for L in lens:
            nb = -(-L // 16)
            bt = (torch.arange(S * nb, device=device, dtype=torch.int32) % (nb_total - 1) + 1).view(S, nb)
            meta = AttentionMetadata(
                query_start_loc=torch.arange(S + 1, device=device, dtype=torch.int32),
                seq_lens=torch.full((S,), L, device=device, dtype=torch.int32), block_tables=bt,
                slot_mapping=torch.zeros(S, device=device, dtype=torch.int64), num_decode=S,
                max_query_len=1, max_seq_len=L)
            q = torch.randn(S, H, D, generator=g, device=device).half()
            cands = [("v2", 0)] + [("v3", p) for p in DECODE_PARTITIONS if p == 0 or p < L]
            best = None
            for (ver, part) in cands:
                t = timer(torch, lambda ver=ver, part=part: K_.paged_attention(
                    q, kc, vc, meta, D ** -0.5, decode_version=ver, partition=part))
                if best is None or t < best[0]:
                    best = (t, ver, part)
            table.set("decode", (S, L), {"version": best[1], "partition": best[2],
                                         "us": round(best[0] * 1e3, 2)})
    return table


def tune(torch, cfg, max_num_seqs: int, max_model_len: int, max_num_batched_tokens: int,
         device="cuda", quantized: bool = True) -> VariantTable:
    """Measure the decode and (when quantized) W8A16 buckets of this model on this GPU."""
    from turingserve_amd import _native

    table = VariantTable(meta={"gpu": torch.cuda.get_device_name(device),
                               "cus": _native.cu_count(torch.device(device).index or 0),
                               "lib": _native.version(), "torch": torch.__version__})
    seqs = [s for s in _ladder(1, 256) if s <= max_num_seqs]
    lens = _ladder(256, max(256, max_model_len))
    tune_decode(torch, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, seqs, lens, device, table)
    if quantized:
        D = cfg.head_dim
        shapes = sorted({(cfg.qkv_dim, cfg.hidden_size), (cfg.hidden_size, cfg.num_heads * D),
                         (2 * cfg.intermediate_size, cfg.hidden_size),
                         (cfg.hidden_size, cfg.intermediate_size)})
        ms = [m for m in W8A16_M_BUCKETS if m < max_num_batched_tokens] + [max_num_batched_tokens]
        tune_w8a16(torch, shapes, ms, device, table)
    return table


def main(argv=None) -> int:
    """Tune this GPU for a model configuration and write the table:
        python -m turingserve_amd.tuner --model qwen2.5-1.5b --out <dir> [--max-num-seqs 64]
            [--max-model-len 4096] [--max-num-batched-tokens 560] [--w8a16-only]"""
    import argparse

    import torch

    from turingserve_amd import _native
    from turingserve_amd.qwen2 import QWEN25_15B, TINY_G2, TINY_G7

    models = {"qwen2.5-1.5b": QWEN25_15B, "tiny-g2": TINY_G2, "tiny-g7": TINY_G7}
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", choices=sorted(models), default="qwen2.5-1.5b")
    ap.add_argument("--out", required=True)
    ap.add_argument("--max-num-seqs", type=int, default=64)
    ap.add_argument("--max-model-len", type=int, default=4096)
    ap.add_argument("--max-num-batched-tokens", type=int, default=560)
    ap.add_argument("--w8a16-only", action="store_true")
    a = ap.parse_args(argv)
    cfg = models[a.model]
    dev = "cuda"
    if a.w8a16_only:
        table = VariantTable(meta={"gpu": torch.cuda.get_device_name(dev)})
        D = cfg.head_dim
        shapes = sorted({(cfg.qkv_dim, cfg.hidden_size), (cfg.hidden_size, cfg.num_heads * D),
                         (2 * cfg.intermediate_size, cfg.hidden_size),
                         (cfg.hidden_size, cfg.intermediate_size)})
        ms = [m for m in W8A16_M_BUCKETS if m < a.max_num_batched_tokens] + [a.max_num_batched_tokens]
        tune_w8a16(torch, shapes, ms, dev, table)
    else:
        table = tune(torch, cfg, a.max_num_seqs, a.max_model_len, a.max_num_batched_tokens, dev)
    name = cache_file_name(torch.cuda.get_device_name(dev), _native.cu_count(0), a.model,
                           _native.version(), torch.__version__)
    print(store_table(a.out, name, table), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
