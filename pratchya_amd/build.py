"""Build the gfx950 shared library ``pratchya_amd/libpratchya_fp8.so``.

The library is built in-tree with ``hipcc --offload-arch=gfx950`` so that it
travels with the source tree to the GPU machine.  Usage::

    python -m pratchya_amd.build          # or pratchya_amd.build.build()
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libpratchya_fp8.so"
SOURCES = ["quantize.hip", "quantize_t.hip", "gemm.hip", "optim.hip", "elementwise.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l)  # host pass does not know the feature
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    objs = []
    build_dir = PKG / "_build"
    build_dir.mkdir(exist_ok=True)
    for src in SOURCES:
        path = CSRC / src
        obj = build_dir / (path.stem + ".o")
        out = _run([HIPCC, *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(path), "-o", str(obj)])
        if verbose and out.strip():
            print(out)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
