"""Compiles generated HIP sources to gfx950 code objects, cached by content
(the reference's compile-once-per-layout-key, ``lumen/runtime/kernel/cuda/driver.rs:148-179``).

The cache lives in ``lumen_amd/_kcache/`` inside the package, so code objects built here on the CPU travel
with the repository to the GPU box; a miss there compiles with the same hipcc.

A code object's key covers everything that decides its bits: the architecture, the flags, the hipcc
version, the generated source and the text of every ``csrc/`` header it includes, transitively. Objects are
filed under a directory named by the hash of that header set (``_kcache/<headers>/<key>.hsaco``), so an
edit to a header leaves its old objects in a directory no current key names, and ``prune()`` removes them.
"""

from __future__ import annotations

import concurrent.futures
import functools
import hashlib
import os
import re
import shutil
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CACHE = os.path.join(os.path.dirname(HERE), "_kcache")
CSRC = os.path.join(os.path.dirname(HERE), "csrc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-variable", "-Wno-unused-but-set-variable"]
_INCLUDE = re.compile(r'^\s*#\s*include\s+"([^"]+)"', re.M)


def hipcc():
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if p and os.path.exists(p):
            return p
    return "hipcc"


VERSION_FILE = os.path.join(CACHE, "HIPCC_VERSION")


def query_hipcc_version() -> str:
    """Runs ``hipcc --version`` (a child process: only before the GPU is initialised) and records the text in
    the cache directory, where later processes read it instead of running the compiler."""
    try:
        r = subprocess.run([hipcc(), "--version"], capture_output=True, text=True, timeout=120)
        text = "\n".join(r.stdout.splitlines()[:2])
    except (OSError, subprocess.SubprocessError):
        return "unknown"
    os.makedirs(CACHE, exist_ok=True)
    with open(VERSION_FILE + ".tmp", "w") as f:
        f.write(text)
    os.replace(VERSION_FILE + ".tmp", VERSION_FILE)
    return text


@functools.lru_cache(maxsize=None)
def hipcc_version() -> str:
    """The compiler's own version text (part of every key: a new compiler makes new objects). Read from the
    file the build wrote, so that a process that has initialised the GPU starts no child process for it."""
    try:
        with open(VERSION_FILE) as f:
            return f.read()
    except OSError:
        return query_hipcc_version()


def includes(text: str, csrc: str = CSRC) -> list:
    """The quoted includes of ``text`` that resolve to files under ``csrc``, transitively, in first-seen
    order (a cycle or a repeated header is visited once)."""
    seen, order, todo = set(), [], list(_INCLUDE.findall(text))
    while todo:
        name = todo.pop(0)
        path = os.path.normpath(os.path.join(csrc, name))
        if path in seen or not os.path.isfile(path):
            continue
        seen.add(path)
        order.append(path)
        with open(path) as f:
            todo.extend(_INCLUDE.findall(f.read()))
    return order


def header_digest(source: str, csrc: str = CSRC) -> str:
    h = hashlib.sha256()
    for path in includes(source, csrc):
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    return h.hexdigest()[:16]


def path_for(source: str, csrc: str = CSRC, cache: str = CACHE) -> str:
    headers = header_digest(source, csrc)
    key = "\0".join([ARCH, " ".join(FLAGS), hipcc_version(), headers, source])
    h = hashlib.sha256(key.encode()).hexdigest()[:24]
    return os.path.join(cache, headers, f"{h}.hsaco")


def live_dirs(csrc: str = CSRC) -> set:
    """Header-set directories the current sources can name: one per csrc header taken as the root include,
    plus the one of a source that includes none of them."""
    names = {header_digest("")}
    for f in sorted(os.listdir(csrc)):
        if f.endswith(".h"):
            names.add(header_digest(f'#include "{f}"\n', csrc))
    return names


def prune(csrc: str = CSRC, cache: str = CACHE) -> int:
    """Removes cached objects built against headers that have since changed (and files from the older flat
    layout); returns how many entries were removed."""
    if not os.path.isdir(cache):
        return 0
    keep, removed = live_dirs(csrc), 0
    for name in os.listdir(cache):
        p = os.path.join(cache, name)
        if (os.path.isdir(p) and name in keep) or p == VERSION_FILE:
            continue
        removed += 1
        if os.path.isdir(p):
            shutil.rmtree(p, ignore_errors=True)
        else:
            os.remove(p)
    return removed


def compile_source(source: str) -> str:
    """The code object of ``source`` (compiled on a cache miss)."""
    out = path_for(source)
    if os.path.exists(out):
        return out
    os.makedirs(os.path.dirname(out), exist_ok=True)
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
