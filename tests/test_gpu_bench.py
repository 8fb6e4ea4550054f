"""bench.py --all-configs on the GPU for two small benchmark configurations:
one JSON line each with the fields the measurement tables are built from."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_all_configs_lines():
    print("case: bench.py --all-configs --config C1 --config C5-D32-fp16", flush=True)
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--all-configs", "--config", "C1",
                        "--config", "C5-D32-fp16", "--no-cpu-baseline", "--steps", "3"],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [json.loads(ln) for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert [d["config"] for d in lines] == ["C1", "C5-D32-fp16"]
    c1, c5 = lines
    assert c1["pass"] == "fwd" and c1["bwd_ms"] is None and c1["fwd_ms"] > 0 and c1["tflops"] > 0
    assert c5["pass"] == "fwd+bwd" and c5["bwd_ms"] > 0 and c5["dropout_p"] == 0.1
    assert c5["dropout_mask"].startswith("keep bits")
