"""The C-ABI shim (flash-attn-v100_amd/csrc/fa_abi.cpp) built with host
AddressSanitizer and UndefinedBehaviorSanitizer against recording stub
launchers (tests/sanitize/), and driven through its validation and
parameter-building paths (tests/sanitize/abi_driver.cpp): every dtype, head
dim, bias, dropout and dbias form, every rejection, and sizes and strides that
would overflow careless integer arithmetic.  Host code only: the device part
of the shim (the static scratch array) is compiled but not sanitized, and no
GPU is touched."""
import os
import shutil
import subprocess
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "flash-attn-v100_amd", "csrc")
SAN_DIR = os.path.join(REPO, "tests", "sanitize")
HIPCC = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else shutil.which("hipcc")

# every -fsanitize= goes to the host compiler only
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


@pytest.mark.skipif(HIPCC is None, reason="hipcc not available")
def test_abi_shim_under_asan_and_ubsan():
    inc = ["-I", os.path.join(REPO, "include"), "-I", CSRC, "-I", SAN_DIR]
    base = [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17"] + SAN + inc
    with tempfile.TemporaryDirectory() as d:
        objs = []
        for src in (os.path.join(CSRC, "fa_abi.cpp"), os.path.join(SAN_DIR, "stub_launchers.cpp"),
                    os.path.join(SAN_DIR, "abi_driver.cpp")):
            obj = os.path.join(d, os.path.basename(src) + ".o")
            r = subprocess.run(base + ["-x", "hip", "-c", src, "-o", obj], capture_output=True, text=True)
            assert r.returncode == 0, r.stderr
            objs.append(obj)
        exe = os.path.join(d, "driver")
        r = subprocess.run([HIPCC, "--offload-arch=gfx950"] + SAN + ["-o", exe] + objs, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        # the HIP runtime's own allocations are not the shim's: no leak report
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
        r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out
    assert "runtime error" not in out and "AddressSanitizer" not in out, out
    assert ", 0 failed" in out, out
