"""Compile the gfx950 HIP library in-tree: plastax_amd/libplastax_hip.so.

Run as ``python -m plastax_amd.build`` (``__graft_entry__.build()`` calls
:func:`build`). The library has no Python dependency: ctypes loads it.

Flags that carry meaning:

- ``-ffp-contract=off``: no fused multiply-add contraction. Every product and
  sum of the step rounds to float32 on its own, exactly as the reference's
  jnp operations do, so the device trajectory can be compared bit for bit.
- ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed float32
  instructions (their results have been unreliable on this pool).
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libplastax_hip.so"
SOURCES = ("plastax_hip.hip", "structural.hip", "layout.hip")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-fvisibility=hidden",
    "-Wall",
]


def hipcc() -> str:
    """Path of hipcc (ROCm's, or the one on PATH)."""
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source (in parallel, one object each) and link the
    in-tree shared library."""
    sources = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    procs = []
    objs = []
    for src in sources:
        obj = objdir / (src.stem + ".o")
        objs.append(obj)
        cmd = [hipcc(), *compile_flags, "-c", "-I", str(ROOT / "include"), str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for cmd, proc in procs:
        out, _ = proc.communicate()
        if proc.returncode != 0:
            sys.stderr.write(out)
            failed.append(proc.returncode)
    if failed:
        raise RuntimeError(f"hipcc failed with exit code {failed[0]}")
    tmp = LIB.with_suffix(".so.tmp")
    # hipRTC compiles the site programs at run time (plx_site_compile)
    rocm_lib = pathlib.Path(hipcc()).resolve().parent.parent / "lib"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
           f"-L{rocm_lib}", "-lhiprtc", f"-Wl,-rpath,{rocm_lib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc link failed with exit code {proc.returncode}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
