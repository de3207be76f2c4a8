"""Variant-selection table for the HIP kernels: the role of the reference's tuner and tuning cache
(autopilot/tuner.py:56-134, consulted by ops/triton_ops.py:44-86, loaded by autopilot/startup.py:
20-43), for this backend's variants instead of Triton configs.

Each kernel has candidate variants per shape bucket; tune() times every candidate with HIP events
over graph-captured calls and keeps the fastest; the winners are stored in a JSON file keyed by
GPU, CU count, model dimensions and library / torch versions. At run time the ops look their
bucket up, rounding up to the smallest recorded bucket (as lookup_rounded does in the
reference; for W8A16 only M rounds, N and K must match); a miss takes the library's own plan.
tune() records the M buckets below the engine's token budget and the budget itself.

    kernel "decode": key "S,L"   (decode rows, max_seq_len)  -> {"version": "v2" | "v3",
                                                                  "partition": 0 | 256 | ...}
    kernel "w8a16":  key "N,K,M" (out features, in features, rows) -> {"variant": 0..4,
                                                                  "splits": 0..}

W8A16 variants (ts_w8a16_gemm_v): 0 the library's plan, 1 weight streaming (M <= 32),
2 128 x 64 wide tiles, 3 128 x 128 wide tiles, 4 128 x 32 wide tiles (128 x 64 in the fused
gated-MLP product); splits 0 = the variant's own rule. Decode:
v2 (one workgroup per sequence and KV head group) or v3 with partition 0 (balanced split) or a
fixed partition in tokens. Every variant computes the same result up to fp32 summation order.
"""

from __future__ import annotations

import json
import os
import re
from dataclasses import dataclass, field

W8A16_M_BUCKETS = (1, 8, 16, 32, 64, 128, 256, 512, 768, 1024, 2048, 4096)
DECODE_PARTITIONS = (0, 256, 512, 1024)


def pow2_buckets(lo: int, hi: int) -> list[int]:
    out, v = [], lo
    while v < hi:
        out.append(v)
        v *= 2
    out.append(hi)
    return out


def round_up_bucket(buckets, value: int) -> int:
    for b in buckets:
        if value <= b:
            return b
    return buckets[-1]


def cache_key(gpu: str, cus: int, model: str, lib_version: str, torch_version: str) -> str:
    safe = lambda s: re.sub(r"[^A-Za-z0-9_.+-]", "-", s)  # noqa: E731
    return f"{safe(gpu)}__cu{cus}__{safe(model)}__{safe(lib_version)}__torch{safe(torch_version)}.json"


@dataclass
class VariantTable:
    """kernel -> {bucket key "a,b,..": choice}; meta carries the cache key fields."""

    tables: dict[str, dict[str, dict]] = field(default_factory=dict)
    meta: dict = field(default_factory=dict)

    def set(self, kernel: str, key: tuple[int, ...], choice: dict) -> None:
        self.tables.setdefault(kernel, {})[",".join(str(k) for k in key)] = choice

    def lookup(self, kernel: str, key: tuple[int, ...]) -> dict | None:
        """The choice of the smallest recorded bucket that is >= key in every dimension (exact
        match on leading dimensions that are not sizes is the caller's business: W8A16 keys put
        N and K first, which only ever match exactly). None on a miss."""
        table = self.tables.get(kernel)
        if not table:
            return None
        best = None
        for name, choice in table.items():
            dims = tuple(int(x) for x in name.split(","))
            if len(dims) == len(key) and all(d >= k for d, k in zip(dims, key)) \
                    and (best is None or dims < best[0]):
                best = (dims, choice)
        return best[1] if best else None

    def to_json(self) -> str:
        return json.dumps({"tables": self.tables, "meta": self.meta}, indent=1, sort_keys=True)

    @classmethod
    def from_json(cls, text: str) -> "VariantTable":
        d = json.loads(text)
        if not isinstance(d.get("tables"), dict):
            raise ValueError("variant table without 'tables'")
        return cls(tables=d["tables"], meta=d.get("meta", {}))


ACTIVE = VariantTable()          # consulted by hip_ops


def set_active(table: VariantTable) -> None:
    global ACTIVE
    ACTIVE = table


def w8a16_choice(N: int, K: int, M: int) -> tuple[int, int]:
    """(variant, splits) for a W8A16 product: the choice recorded for this N and K at the
    smallest recorded M >= M, or the library's own plan (0, 0)."""
    table = ACTIVE.tables.get("w8a16")
    if not table:
        return 0, 0
    best = None
    for name, choice in table.items():
        n, k, m = (int(v) for v in name.split(","))
        if n == N and k == K and m >= M and (best is None or m < best[0]):
            best = (m, choice)
    if best is None:
        return 0, 0
    c = best[1]
    variant, splits = int(c["variant"]), int(c["splits"])
    if variant == 1 and M > 32:                     # streaming exists for M <= 32 only
        return 0, 0
    return variant, splits


def decode_choice(S: int, max_seq_len: int) -> tuple[str | None, int | None]:
    """(version, partition) for S decode rows at this max_seq_len, or (None, None)."""
    c = ACTIVE.lookup("decode", (S, max_seq_len))
    if c is None:
        return None, None
    return c["version"], int(c["partition"])


def load_cache(tuning_dir: str, key: str) -> VariantTable | None:
    path = os.path.join(os.path.expanduser(tuning_dir), key)
    try:
        with open(path, encoding="utf-8") as f:
            return VariantTable.from_json(f.read())
    except (OSError, ValueError, KeyError, TypeError, json.JSONDecodeError):
        return None                                 # missing or corrupt -> tune again


def save_cache(tuning_dir: str, key: str, table: VariantTable) -> str:
    d = os.path.expanduser(tuning_dir)
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, key)
    tmp = path + ".tmp"
    with open(tmp, "w", encoding="utf-8") as f:
        f.write(table.to_json())
    os.replace(tmp, path)
    return path


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
    cands = [(0, 0), (2, 0), (2, 1), (2, 2), (2, 4), (3, 0), (3, 2), (4, 0), (4, 2)]
    if M <= 32:
        cands += [(1, 0), (1, 1), (1, 2), (1, 4)]
    return cands


def tune_w8a16(torch, shapes, ms, device="cuda", table: VariantTable | None = None,
               timer=time_call) -> VariantTable:
    """Time every W8A16 candidate for each (N, K) in `shapes` at each M in `ms` (bucket
    values); keep the fastest (ties go to the earlier candidate, the library's plan first)."""
    from turingserve_amd import hip_ops as K_

    table = table or VariantTable()
    g = torch.Generator(device=device).manual_seed(0)
    for (N, K) in shapes:
        wq = torch.randint(-127, 128, (N, K), generator=g, device=device, dtype=torch.int8)
        sc = torch.rand(N, generator=g, device=device) / 127 + 1e-4
        for M in ms:
            x = torch.randn(M, K, generator=g, device=device).half()
            best = None
            for (v, s) in w8a16_candidates(M):
                t = timer(torch, lambda v=v, s=s: K_.w8a16_linear(x, wq, sc, None, cfg=(v, s)))
                if best is None or t < best[0]:
                    best = (t, v, s)
            table.set("w8a16", (N, K, M), {"variant": best[1], "splits": best[2],
                                           "us": round(best[0] * 1e3, 2)})
    return table


def tune_decode(torch, H: int, KVH: int, D: int, seqs, lens, device="cuda",
                table: VariantTable | None = None, timer=time_call) -> VariantTable:
    """Time v2 and v3 (balanced and fixed partitions) for S decode rows of length L each."""
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
    seqs = [s for s in pow2_buckets(1, 256) if s <= max_num_seqs]
    lens = pow2_buckets(256, max(256, max_model_len))
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
    key = cache_key(torch.cuda.get_device_name(dev), _native.cu_count(0), a.model,
                    _native.version(), torch.__version__)
    print(save_cache(a.out, key, table), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
