"""The C ABI's host code (argument checks, path queries, launch plans, the range audit of
every lowrank plan) under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

`python dynamic-conv1d_amd/build.py --host-sanitize` builds libdynconv_hostsan.so: the
host pass of every unit with -fsanitize=address,undefined (-fno-sanitize-recover, so a
finding aborts), the device code as usual.  This test runs test_capi_host.py and
test_api_host.py against that build in a child process with clang's ASan runtime
preloaded (Python itself is not instrumented).  It skips when the build or the runtime
is absent; the GPU is never touched.
"""

import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_LIB = os.path.join(ROOT, "dynamic-conv1d_amd", "dynconv", "libdynconv_hostsan.so")


def _asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


@pytest.mark.skipif(not os.path.exists(SAN_LIB), reason="libdynconv_hostsan.so not built (build.py --host-sanitize)")
@pytest.mark.skipif(_asan_runtime() is None, reason="clang ASan runtime not found")
def test_host_code_under_sanitizers():
    env = dict(os.environ)
    env.update(LD_PRELOAD=_asan_runtime(), DYNCONV_LIB=SAN_LIB, ASAN_OPTIONS="detect_leaks=0",
               UBSAN_OPTIONS="print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
           os.path.join(ROOT, "tests", "test_capi_host.py"), os.path.join(ROOT, "tests", "test_api_host.py")]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out, out[-2000:]
