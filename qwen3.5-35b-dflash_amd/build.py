"""Build recipe for ``libdflash_hip.so`` (hand-written HIP for gfx950 only).

``python build.py`` from this directory, or ``build()`` from Python.  Each
translation unit is compiled in parallel with hipcc, then linked into one
shared library next to this file; the library is replaced atomically.
``python build.py --timeline`` (``build(timeline=True)``) builds the profiling
variant ``libdflash_hip_timeline.so`` instead: the same kernels with phase
timestamps (``-DDFLASH_TIMELINE``), loaded only by ``timeline.py``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY = PACKAGE_DIR / "libdflash_hip.so"
TIMELINE_LIBRARY = PACKAGE_DIR / "libdflash_hip_timeline.so"
SOURCES = ("csrc/api.hip", "csrc/route.hip", "csrc/w4_gemm.hip", "csrc/w4_stream.hip",
           "csrc/w4_tile.hip", "csrc/w4_verify.hip", "csrc/w4_small.hip",
           "csrc/repack.hip")
ARCH = "gfx950"
FLAGS = (
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # keep the compiler from forming packed-fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build libdflash_hip.so")
    return path


def build(verbose: bool = False, timeline: bool = False) -> Path:
    hipcc = _hipcc()
    target = TIMELINE_LIBRARY if timeline else LIBRARY
    flags = (*FLAGS, "-DDFLASH_TIMELINE") if timeline else FLAGS
    with tempfile.TemporaryDirectory(prefix="dflash_build_") as tmp:
        objects, procs = [], []
        for src in SOURCES:
            obj = Path(tmp) / (Path(src).stem + ".o")
            cmd = [hipcc, *flags, "-c", str(PACKAGE_DIR / src), "-o", str(obj)]
            objects.append(obj)
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        for cmd, proc in procs:
            out, _ = proc.communicate()
            if proc.returncode:
                raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
            if verbose and out.strip():
                print(out)
        staged = Path(tmp) / target.name
        link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(staged)]
        proc = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if proc.returncode:
            raise RuntimeError(f"link failed: {' '.join(link)}\n{proc.stdout}")
        tmp_target = target.with_suffix(".so.tmp")
        shutil.copyfile(staged, tmp_target)
        os.replace(tmp_target, target)
    return target


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, timeline="--timeline" in sys.argv))
