"""Builds libnhip.so (the native runtime and built-in kernels) for gfx950 with hipcc.

``python -m lumen_amd.build`` or ``__graft_entry__.build()``. Host code is C++17, device code HIP for gfx950
only; packed FP32 instructions are disabled and FMA contraction is off (exact rounding of fused code).
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libnhip.so")
SOURCES = ["runtime.cpp", "kernels.hip", "attention.hip"]
# Per-source flags. The flash backward's dK/dV kernel holds ~330 registers (one wave a SIMD); with MFMA
# results in VGPRs the allocator keeps the K/V operands in AGPRs instead of shuttling the dK/dV accumulators
# between AGPRs and VGPRs on every tile.
EXTRA = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-shared",
    "-std=c++17",
    "-ffp-contract=off",
    "-Wno-unused-result",
    "-Wl,--no-undefined",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def build(verbose=False):
    """Compiles libnhip.so from csrc/ (always: this is the build check)."""
    from lumen_amd.compiler.kcache import hipcc

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    procs, objs = [], []
    for src in SOURCES:  # one translation unit a process, in parallel
        obj = os.path.join(objdir, src + ".o")
        objs.append(obj)
        cmd = [hipcc()] + FLAGS + EXTRA.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    errors = []
    for src, p in procs:
        _, err = p.communicate()
        if p.returncode != 0:
            errors.append(f"{src}:\n{err[-6000:]}")
    if errors:
        raise RuntimeError("libnhip build failed:\n" + "\n".join(errors))
    cmd = [hipcc()] + FLAGS + objs + ["-o", OUT + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("libnhip link failed:\n" + r.stderr[-6000:])
    os.replace(OUT + ".tmp", OUT)
    if verbose:
        print("built", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
