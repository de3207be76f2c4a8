"""The variant-selection table on the CPU (the role of the reference's tuning cache,
autopilot/tuner.py:56-134): JSON round trip, round-up bucket lookup, the choices the ops take from
it, the cache files, and the library's variant-aware size function."""

from __future__ import annotations

import ctypes

import pytest

from turingserve_amd import _native as N
from turingserve_amd import tuner as T


@pytest.fixture(autouse=True)
def _restore_active():
    saved = T.ACTIVE
    yield
    T.set_active(saved)


def test_table_round_trip_and_round_up_lookup():
    t = T.VariantTable(meta={"gpu": "x"})
    t.set("decode", (4, 1024), {"version": "v3", "partition": 0})
    t.set("decode", (4, 4096), {"version": "v3", "partition": 512})
    t.set("decode", (64, 1024), {"version": "v2", "partition": 0})
    u = T.VariantTable.from_json(t.to_json())
    assert u.records("decode") == t.records("decode") and u.meta == {"gpu": "x"}
    assert u.to_json() == t.to_json()
    assert u.lookup("decode", (3, 900)) == {"version": "v3", "partition": 0}
    assert u.lookup("decode", (4, 1025)) == {"version": "v3", "partition": 512}
    assert u.lookup("decode", (5, 100)) == {"version": "v2", "partition": 0}
    assert u.lookup("decode", (65, 100)) is None and u.lookup("w8a16", (1, 1, 1)) is None
    with pytest.raises(ValueError):
        T.VariantTable.from_json('{"tables": {}}')            # another layout


def test_choices_follow_the_active_table():
    assert T.w8a16_choice(2048, 1536, 560) == (0, 0)          # empty table: the library's plan
    assert T.decode_choice(8, 4096) == (None, None)
    t = T.VariantTable()
    t.set("w8a16", (2048, 1536, 768), {"variant": 2, "splits": 2})
    t.set("w8a16", (2048, 1536, 32), {"variant": 1, "splits": 4})
    t.set("w8a16", (2048, 1536, 64), {"variant": 1, "splits": 1})
    t.set("decode", (8, 4096), {"version": "v3", "partition": 256})
    T.set_active(t)
    assert T.w8a16_choice(2048, 1536, 560) == (2, 2)          # 560 rounds up to the 768 bucket
    assert T.w8a16_choice(2048, 1536, 20) == (1, 4)
    assert T.w8a16_choice(2048, 1536, 32) == (1, 4)
    assert T.w8a16_choice(2048, 1536, 40) == (0, 0)           # streaming cannot take M = 40
    assert T.w8a16_choice(2048, 1536, 1000) == (0, 0)         # bucket 1024 not recorded
    assert T.w8a16_choice(1536, 1536, 560) == (0, 0)          # other shape
    assert T.decode_choice(5, 3000) == ("v3", 256)


def test_cache_files(tmp_path):
    name = T.cache_file_name("AMD Instinct MI355X", 256, "qwen2.5-1.5b/int8",
                             "turingserve_hip 0.1.0", "2.10.0+rocm7.0")
    assert "/" not in name and " " not in name and name.endswith(".json")
    assert name != T.cache_file_name("AMD Instinct MI355X", 256, "qwen2.5-1.5b/int8",
                                     "turingserve_hip 0.1.1", "2.10.0+rocm7.0")
    t = T.VariantTable()
    t.set("w8a16", (8, 8, 1), {"variant": 3, "splits": 1})
    path = T.store_table(str(tmp_path), name, t)
    assert T.load_table(str(tmp_path), name).records("w8a16") == t.records("w8a16")
    assert sorted(p.name for p in tmp_path.iterdir()) == [name]     # no temporary left behind
    open(path, "w").write("{not json")
    assert T.load_table(str(tmp_path), name) is None
    assert T.load_table(str(tmp_path), "missing.json") is None


def test_variant_workspace_sizes_and_checks():
    lib = N.lib()
    for shape in ((560, 1536, 8960), (1, 2048, 1536), (2048, 17920, 1536)):
        assert lib.ts_w8a16_workspace_bytes_v(*shape, 0, 0, 256) == \
            lib.ts_w8a16_workspace_bytes(*shape, 256)
    assert lib.ts_w8a16_workspace_bytes_v(560, 1536, 1536, 2, 2, 256) == 2 * 560 * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes_v(560, 1536, 1536, 3, 1, 256) == 0
    assert lib.ts_w8a16_workspace_bytes_v(560, 1536, 1536, 4, 0, 256) == 0   # 128 x 32: no split
    assert lib.ts_w8a16_workspace_bytes_v(560, 1536, 1536, 4, 3, 256) == 3 * 560 * 1536 * 4
    assert lib.ts_w8a16_glu_workspace_bytes(560, 768, 1536, 4, 2, 256) == 2 * 560 * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes_v(8, 1536, 1536, 1, 3, 256) == 3 * 8 * 1536 * 4
    assert lib.ts_w8a16_workspace_bytes_v(64, 1536, 1536, 1, 0, 256) == 0    # not available
    p = ctypes.c_void_p(256)
    st = lib.ts_w8a16_gemm_v(p, 1536, p, p, 0, None, p, 1536, 64, 1536, 1536, 1, 0, None, 0, None)
    assert st == N.TS_ERR_UNSUPPORTED and "variant 1" in N.last_error()
    st = lib.ts_w8a16_gemm_v(p, 1536, p, p, 0, None, p, 1536, 8, 1536, 1536, 7, 0, None, 0, None)
    assert st == N.TS_ERR_UNSUPPORTED
