import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "flash-attn-v100_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running (full-size benchmark configs C1-C5)")


def _ensure_built():
    lib = os.path.join(PKG_ROOT, "flash_attention_v100", "libfa_gfx950.so")
    if not os.path.exists(lib):
        subprocess.run([sys.executable, os.path.join(PKG_ROOT, "build.py")], check=True)
    olib = os.path.join(REPO, "oracle", "_build", "liboracle.so")
    if not os.path.exists(olib):
        subprocess.run(["make", "-C", os.path.join(REPO, "oracle")], check=True,
                       stdout=subprocess.DEVNULL)


_ensure_built()
