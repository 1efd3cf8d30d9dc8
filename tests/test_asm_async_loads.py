"""The three-buffer integer-dot matrix-core matvec (matvec_i8_mfma with NB = 3, sharplight_amd/csrc/matvec_i8.hpp)
loads each stage's q8 values into registers with inline-assembly global loads that the compiler does not track:
nothing may read or write a register such a load writes before an `s_waitcnt vmcnt` has retired the load (a
spill of the register, a copy of part of it, or its reuse for another value would see or clobber stale data).
This test compiles the formats that take three buffers to gfx950 assembly and checks their kernels by modelling
the in-order vmcnt queue over each kernel's instruction stream. Runs on the CPU (hipcc cross-compiles)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "sharplight_amd", "csrc")
BUILD = os.path.join(ROOT, "sharplight_amd", "_build")

VM_OP = re.compile(r"(global_load\w*|buffer_load\w*|flat_load\w*|global_atomic\w*)\b")
VREG = re.compile(r"v\[\d+:\d+\]|v\d+\b")


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def pending_load_hazards(lines):
    """Instructions that touch the destination of a vector-memory load still counted by vmcnt. The queue is
    retired by `s_waitcnt vmcnt(n)` (all but the newest n); loads into LDS have no register destination."""
    queue, hazards = [], []
    for line in lines:
        s = line.split(";")[0].strip()
        if not s or s.endswith(":") or s.startswith("."):
            continue
        w = re.match(r"s_waitcnt\s+(.*)", s)
        if w:
            m = re.search(r"vmcnt\((\d+)\)", w.group(1))
            if m:
                n = int(m.group(1))
                queue = queue[len(queue) - n:] if n < len(queue) else queue
            continue
        ops = VREG.findall(s)
        vm = VM_OP.match(s)
        dest = _regs(ops[0]) if vm and ops and "lds" not in vm.group(1) else set()
        touched = set()
        for o in (ops[1:] if dest else ops):
            touched |= _regs(o)
        for src, d in queue:
            if d & touched:
                hazards.append((src, s))
                break
        if vm:
            queue.append((s, dest))
    return hazards


def test_checker_sees_an_early_read():
    # the checker itself: a read before the wait is flagged, after it is not, and vmcnt(1) retires the older load
    bad = ["global_load_dwordx2 v[4:5], v[0:1], off", "v_add_u32_e32 v6, v4, v7", "s_waitcnt vmcnt(0)"]
    good = ["global_load_dwordx2 v[4:5], v[0:1], off", "s_waitcnt vmcnt(0)", "v_add_u32_e32 v6, v4, v7"]
    two = ["global_load_dwordx2 v[4:5], v[0:1], off", "global_load_dwordx2 v[8:9], v[0:1], off",
           "s_waitcnt vmcnt(1)", "v_add_u32_e32 v6, v4, v7", "v_add_u32_e32 v6, v8, v7"]
    reuse = ["global_load_dwordx4 v[2:5], v[0:1], off", "v_cndmask_b32_e64 v4, 0, 1, s[2:3]"]
    assert len(pending_load_hazards(bad)) == 1
    assert pending_load_hazards(good) == []
    assert [h[1] for h in pending_load_hazards(two)] == ["v_add_u32_e32 v6, v8, v7"]
    assert len(pending_load_hazards(reuse)) == 1


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return None


def test_three_buffer_kernels_wait_for_their_register_loads(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    if not os.path.exists(os.path.join(BUILD, "ewg_jit_sources.inc")):
        pytest.skip("run the library build first (it writes the generated include)")
    # only the formats whose I8Stage takes three buffers, instantiated on their own (the format files would
    # compile every kernel of three formats)
    hpp = open(os.path.join(CSRC, "matvec_i8.hpp")).read()
    fmts = re.findall(r"struct I8Stage<(SLHIP_FMT_\w+)> \{[^}]*NB = 3", hpp)
    assert fmts, "no format takes three buffers"
    src = tmp_path / "nb3.hip"
    src.write_text('#include "matvec_i8.hpp"\nnamespace slhip {\n' + "".join(
        f"template int run_i8_mfma<{f}>(I8Args, bool, hipStream_t);\n" for f in fmts) + "}\n")
    out = tmp_path / "nb3.s"
    r = subprocess.run([hipcc, "-O3", "-std=c++17", "--offload-arch=gfx950", "--cuda-device-only", "-S",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", BUILD, "-I", CSRC,
                        "-o", str(out), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    text = out.read_text()
    checked = 0
    # kernels matvec_i8_mfma<FMT, DUAL, SU, TN, NB = 3>
    for m in re.finditer(r"\n(_ZN5slhip14matvec_i8_mfma\w+Li3EEEvNS_6I8ArgsE):[^\n]*\n(.*?)\n\s*s_endpgm", text, re.S):
        hz = pending_load_hazards(m.group(2).split("\n"))
        assert hz == [], f"{m.group(1)}: {hz[:3]}"
        checked += 1
    assert checked == 2 * len(fmts), f"{checked} three-buffer kernels found for {fmts}"
