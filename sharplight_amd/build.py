"""Builds libsharplight_hip.so in-tree with hipcc for gfx950.

Each ``csrc/*.hip`` compiles to an object under ``sharplight_amd/_build/`` (in parallel), then one link
produces ``sharplight_amd/libsharplight_hip.so``. ``python -m sharplight_amd.build`` runs it.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsharplight_hip.so")
# GPU check programs of the test suite (sources under tests/, binaries beside them under tests/_bin/)
TESTS = os.path.join(os.path.dirname(HERE), "tests")
CHECKS = ["e4m3_exhaustive", "recip_exhaustive"]
ARCH = os.environ.get("SLHIP_ARCH", "gfx950")

# Packed-f32 VALU forms are disabled: hipcc -O3 would otherwise form them from plain float code.
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-fvisibility=hidden",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-command-line-argument"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _includes(path: str, seen: set) -> None:
    """Adds the csrc/ and include/ headers that path includes, transitively, to seen."""
    import re
    try:
        text = open(path).read()
    except OSError:
        return
    for name in re.findall(r'#include\s+"([^"]+)"', text):
        for base in (os.path.dirname(path), CSRC, os.path.join(os.path.dirname(HERE), "include")):
            cand = os.path.normpath(os.path.join(base, name))
            if os.path.exists(cand):
                if cand not in seen:
                    seen.add(cand)
                    _includes(cand, seen)
                break


def _stale(src: str, obj: str) -> bool:
    """Whether obj is older than src or than any header src includes (directly or through other headers)."""
    if not os.path.exists(obj):
        return True
    deps = {src}
    _includes(src, deps)
    return max(os.path.getmtime(d) for d in deps) > os.path.getmtime(obj)


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if incremental and not _stale(src, obj):
        return obj
    cmd = [hipcc(), *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compiles every source (incremental: only those whose object is older than the source or a header)."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda src: _compile(src, incremental), sources))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    # a host pass that drops a kernel's launch stub still exits 0: refuse a library with undefined own symbols
    nm = subprocess.run(["nm", "-D", "--undefined-only", tmp], capture_output=True, text=True)
    missing = [l.split()[-1] for l in nm.stdout.splitlines() if "slhip" in l]
    if missing:
        raise RuntimeError(f"link left symbols of this library undefined: {missing[:5]}")
    os.replace(tmp, LIB)
    os.makedirs(os.path.join(TESTS, "_bin"), exist_ok=True)
    for name in CHECKS:
        exe = os.path.join(TESTS, "_bin", name)
        if incremental and not _stale(os.path.join(TESTS, name + ".hip"), exe):
            continue
        r = subprocess.run([hipcc(), *[f for f in CFLAGS if f not in ("-fPIC", "-fvisibility=hidden")], "-o", exe,
                            os.path.join(TESTS, name + ".hip")], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on tests/{name}.hip:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)
