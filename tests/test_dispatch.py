"""The MI355X dispatch tables (prism_amd.dispatch): the reference's lookup rules (kernels/w8a8.py:163-168 nearest
measured token count in log scale; kernels/w4a8.py:309-316 smallest measured count >= M, else the largest), the
environment overrides, and that the committed tables are well formed (every shape a key of the right form, every
choice a kernel its op provides and valid at that token count)."""
import glob
import json
import os

import pytest

from prism_amd import dispatch


@pytest.fixture
def tables(tmp_path, monkeypatch):
    w8 = {"table": {"5120x5120": {"1": ["decode"], "16": ["mid"], "64": ["decode"], "128": ["tile"]}}}
    w4 = {"table": {"q4k,13824,5120": {"1": ["decode"], "16": ["tile"], "2048": ["tile"]}}}
    for name, doc in (("gemm.json", w8), ("q8.json", w8), ("w4.json", w4)):
        (tmp_path / name).write_text(json.dumps(doc))
    monkeypatch.setenv("STARTLUX_PRISM_GEMM_TABLE", str(tmp_path / "gemm.json"))
    monkeypatch.setenv("STARTLUX_PRISM_Q8_TABLE", str(tmp_path / "q8.json"))
    monkeypatch.setenv("STARTLUX_PRISM_W4A8_TABLE", str(tmp_path / "w4.json"))
    dispatch.load.cache_clear()
    yield
    dispatch.load.cache_clear()


def test_w8a8_nearest_in_log_scale(tables):
    assert dispatch.w8a8_kernel(5120, 5120, 1, 32) == "decode"
    assert dispatch.w8a8_kernel(5120, 5120, 3, 32) == "decode"      # |log 3 - log 1| < |log 3 - log 16|
    assert dispatch.w8a8_kernel(5120, 5120, 5, 32) == "mid"         # log 5 is nearer log 16 than log 1
    assert dispatch.w8a8_kernel(5120, 5120, 91, 5120) == "tile"     # 91 > sqrt(64 128) = 90.5: nearer 128
    assert dispatch.w8a8_kernel(5120, 5120, 90, 5120) == "decode"
    assert dispatch.w8a8_kernel(5120, 5120, 9000, 32) == "tile"
    assert dispatch.w8a8_kernel(4096, 5120, 1, 32) == "auto"        # shape not in the table
    assert dispatch.w8a8_kernel(5120, 5120, 1, 64) == "auto"        # no table for other groupings


def test_w4a8_smallest_at_least(tables):
    assert dispatch.w4a8_kernel("q4k", 13824, 5120, 1) == "decode"
    assert dispatch.w4a8_kernel("q4k", 13824, 5120, 2) == "tile"    # next measured count is 16
    assert dispatch.w4a8_kernel("q4k", 13824, 5120, 5000) == "tile"  # beyond the table: its largest
    assert dispatch.w4a8_kernel("q6k", 13824, 5120, 1) == "auto"


def test_off(tables, monkeypatch):
    monkeypatch.setenv("STARTLUX_PRISM_W4A8_TABLE", "off")
    dispatch.load.cache_clear()
    assert dispatch.w4a8_kernel("q4k", 13824, 5120, 1) == "auto"


LIMITS = {"gemm_table": {"decode": 1 << 20, "split": 512, "tile": 1 << 30}, "q8_table": {"decode": 64, "stream": 16, "mid": 1 << 20,
                                                                                   "tile": 1 << 30},
          "w4a8_table": {"decode": 16, "stream": 16, "tile": 1 << 30}}


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(dispatch.HERE, "*_table_*.json"))))
def test_committed_tables_well_formed(path):
    prefix = os.path.basename(path).split("_table_")[0] + "_table"
    doc = json.load(open(path))
    assert doc["gpu"] and doc["source"] and doc["table"]
    for key, row in doc["table"].items():
        parts = key.split(",") if prefix == "w4a8_table" else key.split("x")
        if prefix == "w4a8_table":
            assert parts[0] in ("q4k", "q6k") and int(parts[1]) % 16 == 0 and int(parts[2]) % 256 == 0
        else:
            assert len(parts) == 2 and int(parts[0]) % 16 == 0
        for m, choice in row.items():
            assert choice[0] in LIMITS[prefix] and int(m) <= LIMITS[prefix][choice[0]], (key, m, choice)
            # W4A8 on Q4_K: the balanced stream kernel needs its activation image in LDS (M (K + 32) bytes and the
            # sums, scales and terms, within 160 KB)
            if prefix == "w4a8_table" and choice[0] == "stream" and parts[0] == "q4k":
                M, K = int(m), int(parts[2])
                assert M * (K + 32) + K // 16 * M + K // 64 * M + 3 * 12 * M * 64 + 64 <= 160 * 1024, (key, m)
