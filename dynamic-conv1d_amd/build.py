"""Build libdynconv.so (gfx950) in-tree with hipcc.

    python dynamic-conv1d_amd/build.py [--jobs N] [--host-sanitize]

Each csrc/*.hip translation unit is compiled in parallel to _build/*.o and
linked into dynconv/libdynconv.so.  Always rebuilds (the driver's "does it
build" check calls this on every round).

--host-sanitize builds dynconv/libdynconv_hostsan.so instead (objects in
_build_hostsan/): the host code (argument checks, launch plans, the range
audit) with AddressSanitizer and UndefinedBehaviorSanitizer, the device code
as usual.  It is for CPU runs only: tests/test_host_sanitize.py runs the C-ABI
host tests against it in a child process with clang's ASan runtime preloaded.
"""

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "dynconv", "libdynconv.so")
BUILD_SAN = os.path.join(HERE, "_build_hostsan")
OUT_SAN = os.path.join(HERE, "dynconv", "libdynconv_hostsan.so")
# Sanitizers for the host pass only (each -fsanitize= behind -Xarch_host).
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

ARCH = "gfx950"
# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU ops (v_pk_*_f32).
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
]
# Per-file flags.  The lowrank forward lets its MFMA results land in VGPRs
# directly (no v_accvgpr_read per result); the backward keeps the default,
# where accumulation registers are what keeps its larger tiles in 512 registers.
# lowrank_mfma_fwd_ilp.hip is the forward's one-rank-chunk kernel scheduled
# for instruction-level parallelism (see that file).
PER_FILE = {"lowrank_mfma_fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
            "lowrank_mfma_fwd_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
            "lowrank_mfma_dx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
            "lowrank_mfma_fwd_ilp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-sched-strategy=max-ilp"],
            "lowrank_f32_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libdynconv.so)")


def _compile(src: str, extra: list, bdir: str = BUILD) -> tuple:
    obj = os.path.join(bdir, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *COMMON, *PER_FILE.get(os.path.basename(src), []), *extra, "-c", src, "-o", obj]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    return src, obj, r.returncode, err, time.time() - t0


def build(jobs: int = 0, extra=None, verbose: bool = True, host_sanitize: bool = False) -> str:
    extra = list(extra or []) + (HOST_SAN if host_sanitize else [])
    bdir, out = (BUILD_SAN, OUT_SAN) if host_sanitize else (BUILD, OUT)
    os.makedirs(bdir, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    objs = []
    failed = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, obj, rc, err, dt in ex.map(lambda s: _compile(s, extra, bdir), srcs):
            if verbose:
                print(f"[build] {os.path.basename(src)}: {'ok' if rc == 0 else 'FAILED'} ({dt:.1f}s)", flush=True)
            if err.strip() and (rc != 0 or verbose):
                print(err, file=sys.stderr, flush=True)
            if rc != 0:
                failed.append(src)
            objs.append(obj)
    if failed:
        raise RuntimeError(f"hipcc failed for: {', '.join(os.path.basename(f) for f in failed)}")
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[build] wrote {out}", flush=True)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=0)
    ap.add_argument("--host-sanitize", action="store_true", help="build libdynconv_hostsan.so (ASan + UBSan host code)")
    args = ap.parse_args()
    build(args.jobs, host_sanitize=args.host_sanitize)
