"""bench.py on a machine without a GPU: the multi-GPU refusal, the benchmark
configuration table against BASELINE.json, the FLOP convention and a tiny
CPU-baseline sample."""
import json
import os
import re
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_config_table_matches_baseline_json():
    texts = json.load(open(os.path.join(REPO, "BASELINE.json")))["configs"]
    shapes = [tuple(int(x) for x in m.group(1).split(","))
              for m in (re.search(r"\(B,S,H,D\) = \(([0-9,]+)", t) for t in texts[:4])]
    by_name = {c[0]: c for c in bench.ALL_CONFIGS}
    assert by_name["C1"][1] == shapes[0] and by_name["C1"][2] == "float16" and not by_name["C1"][3]
    assert by_name["C1"][5] is False  # forward only
    assert by_name["C2"][1] == shapes[1] and by_name["C2"][3] and by_name["C2"][5]
    assert by_name["C3"][1] == shapes[2] and by_name["C3"][2] == "bfloat16" and by_name["C3"][3]
    assert by_name["C4-causal"][1] == shapes[3] == by_name["C4-full"][1]
    assert by_name["C4-causal"][3] and not by_name["C4-full"][3]
    assert "(8,1000,16,{32,64,128})" in texts[4] and "dropout_p=0.1" in texts[4]
    c5 = [c for c in bench.ALL_CONFIGS if c[0].startswith("C5")]
    assert sorted((c[1][3], c[2]) for c in c5) == sorted((d, t) for d in (32, 64, 128) for t in ("float32", "float16"))
    assert all(c[1][:3] == (8, 1000, 16) and c[3] and c[4] == 0.1 for c in c5)


def test_flop_convention():
    # F_fwd = 4 B H S^2 D (x 1/2 causal): the headline's 549.76 GFLOP and C4's 2199.0 / 1099.5
    assert bench.f_fwd() == pytest.approx(549.76e9, rel=1e-5)
    assert bench.f_fwd(1, 16, 16384, 128, False) == pytest.approx(2199.0e9, rel=1e-4)
    assert bench.f_fwd(1, 16, 16384, 128, True) == pytest.approx(1099.5e9, rel=1e-4)
    assert bench.f_fwd(2, 12, 1024, 64, False) == pytest.approx(6.442e9, rel=1e-3)


def test_cpu_sample_is_sane():
    r = bench._cpu_sample(64, 2, 32, True, 0.1, True, 0.05)
    assert r["value"] > 0 and r["kind"] == "port" and r["cores"] >= 1 and "oracle.attention" in r["sample"]
