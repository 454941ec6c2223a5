"""bench.py's contract, checked without a GPU: one GPU only, and the
dominant kernel's HBM traffic record belongs to the kernel sources in the
tree (bench.py reports `roofline.traffic` only from a record whose source
hash matches; this keeps the committed record current)."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
    assert p.stdout == ""  # no JSON line


def test_pmc_record_is_this_builds():
    path = os.path.join(ROOT, "profiles", "gemv_gate_up_4b_pmc.json")
    rec = json.load(open(path))
    assert rec["kernel_source_sha256"] == bench.dominant_source_sha(), (
        "gemv.hip or common.hpp changed since the PMC passes: re-run them")
    assert rec["sources"] == [os.path.relpath(p, ROOT) for p in bench.DOM_SOURCES]
    assert rec["bytes"] == bench.dominant_bytes()
    # FETCH_SIZE counts half the bytes on gfx950 (a 256 MiB copy reads as
    # 131,088 KiB), WRITE_SIZE all of them
    assert rec["fetch_factor"] == pytest.approx(2.0, rel=1e-3)
    assert rec["write_factor"] == pytest.approx(1.0, rel=1e-3)
    traffic = (rec["fetch_kib_per_dispatch"] * rec["fetch_factor"] +
               rec["write_kib_per_dispatch"] * rec["write_factor"]) * 1024
    assert traffic == pytest.approx(rec["traffic_bytes"], rel=1e-6)
    assert 1.0 <= rec["traffic_bytes"] / rec["bytes"] < 1.05
