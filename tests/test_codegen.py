"""Code generation guard over the built gfx950 code objects (CPU; no GPU needed).

A buffer resource whose base or byte count the compiler computed on the vector
unit cannot be proven uniform; every access through it then becomes a loop over
the lanes' distinct descriptors (readfirstlane of the four descriptor words, a
64-bit compare per pair, exec narrowed to the matching lanes, the access, the
remaining lanes).  Such loops cost hundreds of instructions per row, and the
register allocator has placed copies at the top of a loop's exit block, before
exec is restored, where they run with no lane enabled: the fp16 W 16 head-size-1
headwise backward lost a dx ring slot that way (rows 16k+15 wrong).  The kernels
build their resources from uniform values (make_rsrc_wave where the compiler
would not see it); this test disassembles every object of the build and fails on
any such loop.
"""

import concurrent.futures as cf
import glob
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "dynamic-conv1d_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# readfirstlane of a descriptor word, then within a few instructions a 64-bit
# equality compare of those SGPRs against the VGPR pair they came from
RFL = re.compile(r"v_readfirstlane_b32\s+(s\d+),\s*(v\d+)")
CMP = re.compile(r"v_cmp_eq_u64\S*\s+\S+,\s*s\[(\d+):\d+\],\s*v\[(\d+):\d+\]")
SYM = re.compile(r"^[0-9a-f]+ <(\S+)>:")


def _tools():
    need = [shutil.which("objcopy"), os.path.join(LLVM, "clang-offload-bundler"), os.path.join(LLVM, "llvm-objdump")]
    return all(p and os.path.exists(p) for p in need)


def _descriptor_loops(obj):
    """Kernels of one object file that contain per-lane descriptor loops: {symbol: count}."""
    with tempfile.TemporaryDirectory() as tmp:
        fb, co = os.path.join(tmp, "fb"), os.path.join(tmp, "co")
        r = subprocess.run(["objcopy", f"--dump-section=.hip_fatbin={fb}", obj, os.path.join(tmp, "o")],
                           capture_output=True, text=True)
        if r.returncode != 0 or not os.path.exists(fb):
            return None  # no device code in this object
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--type=o", f"--targets={TARGET}",
                        f"--input={fb}", f"--output={co}", "--unbundle"], check=True, capture_output=True)
        proc = subprocess.Popen([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", co],
                                stdout=subprocess.PIPE, text=True)
        found, sym, recent = {}, None, []
        for line in proc.stdout:
            m = SYM.match(line)
            if m:
                sym, recent = m.group(1), []
                continue
            m = RFL.search(line)
            if m:
                recent = (recent + [(int(m.group(1)[1:]), int(m.group(2)[1:]))])[-8:]
                continue
            m = CMP.search(line)
            if m and recent:
                s0, v0 = int(m.group(1)), int(m.group(2))
                if any(s == s0 and v == v0 for s, v in recent):
                    found[sym] = found.get(sym, 0) + 1
        proc.wait()
        assert proc.returncode == 0, f"llvm-objdump failed on {obj}"
        return found


def test_no_per_lane_descriptor_loops():
    objs = sorted(glob.glob(os.path.join(BUILD, "*.o")))
    if not objs:
        pytest.skip("no build objects (python dynamic-conv1d_amd/build.py)")
    if not _tools():
        pytest.skip("objcopy / clang-offload-bundler / llvm-objdump not available")
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        results = dict(zip(objs, ex.map(_descriptor_loops, objs)))
    scanned = [o for o, r in results.items() if r is not None]
    assert scanned, "no object carried gfx950 device code"
    bad = {os.path.basename(o): r for o, r in results.items() if r}
    summary = {o: (len(r), sorted(r)[:3]) for o, r in bad.items()}
    assert not bad, f"per-lane buffer-descriptor loops (resources not provably uniform), " \
                    f"object: (kernels, first names): {summary}"


def test_detector_finds_a_descriptor_loop():
    """The pattern matcher on a hand-written loop of the shape the compiler emits."""
    text = """0000000000001000 <kernel>:
	v_readfirstlane_b32 s8, v2
	v_readfirstlane_b32 s9, v3
	v_readfirstlane_b32 s10, v4
	v_readfirstlane_b32 s11, v5
	v_cmp_eq_u64_e32 vcc, s[8:9], v[2:3]
	v_cmp_eq_u64_e64 s[2:3], s[10:11], v[4:5]
	s_and_b64 s[2:3], vcc, s[2:3]
	s_and_saveexec_b64 s[2:3], s[2:3]
	buffer_load_dwordx4 v[16:19], v20, s[8:11], 0 offen
	s_xor_b64 exec, exec, s[2:3]
	s_cbranch_execnz 65528
"""
    hits, recent = 0, []
    for line in text.splitlines():
        m = RFL.search(line)
        if m:
            recent = (recent + [(int(m.group(1)[1:]), int(m.group(2)[1:]))])[-8:]
            continue
        m = CMP.search(line)
        if m and any(s == int(m.group(1)) and v == int(m.group(2)) for s, v in recent):
            hits += 1
    assert hits == 2
