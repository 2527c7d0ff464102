"""Build the gfx950 HIP library in-tree: qw6_amd/libqw6_hip.so.

    python -m qw6_amd.build

All HIP sources are compiled for gfx950 only, with packed-FP32 instruction
selection disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libqw6_hip.so"
SOURCES = ["qw6_hip.hip", "qw6_prefill.hip", "qw6_gguf.cpp", "qw6_selftest.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + str(PKG.parent / "include")]


def build(verbose: bool = False) -> Path:
    """Compile every source to an object in parallel (one hipcc per source),
    then link the shared library."""
    srcs = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    odir = PKG / "_build"
    odir.mkdir(exist_ok=True)
    procs = []
    for s in srcs:
        obj = odir / (s.name + ".o")
        cmd = [HIPCC, *FLAGS, "-c", "-o", str(obj), str(s)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((s, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                               stderr=subprocess.STDOUT, text=True)))
    failed = False
    for s, obj, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            sys.stderr.write(out)
            failed = True
    if failed:
        raise RuntimeError("hipcc failed building %s" % LIB)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-o", str(tmp), *[str(o) for _, o, _ in procs]]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed linking %s" % LIB)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
