"""Compiles generated HIP sources to gfx950 code objects, cached by source hash
(the reference's compile-once-per-layout-key, ``lumen/runtime/kernel/cuda/driver.rs:148-179``).

The cache lives in ``lumen_amd/_kcache/`` inside the package, so code objects built here on the CPU travel
with the repository to the GPU box; a miss there compiles with the same hipcc.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CACHE = os.path.join(os.path.dirname(HERE), "_kcache")
CSRC = os.path.join(os.path.dirname(HERE), "csrc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-variable", "-Wno-unused-but-set-variable"]


def hipcc():
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if p and os.path.exists(p):
            return p
    return "hipcc"


def path_for(source: str) -> str:
    h = hashlib.sha256((ARCH + " ".join(FLAGS) + source).encode()).hexdigest()[:24]
    return os.path.join(CACHE, f"{h}.hsaco")


def compile_source(source: str) -> str:
    """The code object of ``source`` (compiled on a cache miss)."""
    out = path_for(source)
    if os.path.exists(out):
        return out
    os.makedirs(CACHE, exist_ok=True)
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "k.hip")
        with open(src, "w") as f:
            f.write(source)
        tmp = os.path.join(d, "k.hsaco")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "--genco", "-I", CSRC] + FLAGS + [src, "-o", tmp]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on a generated kernel:\n{r.stderr[-4000:]}\n--- source ---\n{source[:6000]}")
        os.replace(tmp, out)
    return out


def compile_many(sources: list, jobs: int | None = None) -> list:
    """Code objects of ``sources``, compiling misses in parallel."""
    jobs = jobs or min(16, os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        return list(ex.map(compile_source, sources))
