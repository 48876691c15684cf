"""The generated-kernel cache key: header edits, the compiler version and the source all change it, and
``prune`` drops objects built against headers that have changed."""

import os
import shutil

from lumen_amd.compiler import kcache


def _csrc_copy(tmp_path):
    d = tmp_path / "csrc"
    shutil.copytree(kcache.CSRC, d)
    return str(d)


def test_key_follows_transitively_included_headers(tmp_path):
    csrc = _csrc_copy(tmp_path)
    src = '#include "gemm.h"\n__global__ void k() {}\n'
    names = [os.path.basename(p) for p in kcache.includes(src, csrc)]
    assert names[:2] == ["gemm.h", "device_common.h"]
    before = kcache.path_for(src, csrc, str(tmp_path / "c"))
    # an edit to a header reached only through gemm.h still changes the key
    with open(os.path.join(csrc, "device_common.h"), "a") as f:
        f.write("\n// edited\n")
    after = kcache.path_for(src, csrc, str(tmp_path / "c"))
    assert after != before
    assert os.path.dirname(after) != os.path.dirname(before)
    # a source with no csrc include is unaffected by header edits
    plain = "__global__ void k() {}\n"
    assert os.path.dirname(kcache.path_for(plain, csrc)) == os.path.dirname(kcache.path_for(plain))


def test_key_covers_source_and_compiler(monkeypatch):
    a = kcache.path_for("__global__ void a() {}\n")
    assert kcache.path_for("__global__ void b() {}\n") != a
    monkeypatch.setattr(kcache, "hipcc_version", lambda: "another compiler")
    assert kcache.path_for("__global__ void a() {}\n") != a


def test_prune_drops_entries_of_changed_headers(tmp_path):
    csrc = _csrc_copy(tmp_path)
    cache = tmp_path / "cache"
    src = '#include "gemm.h"\n'
    old = kcache.path_for(src, csrc, str(cache))
    os.makedirs(os.path.dirname(old))
    open(old, "w").close()
    (cache / "0123456789abcdef.hsaco").write_text("")  # the older flat layout
    assert kcache.prune(csrc, str(cache)) == 1
    assert os.path.exists(old)
    with open(os.path.join(csrc, "gemm.h"), "a") as f:
        f.write("\n// edited\n")
    assert kcache.prune(csrc, str(cache)) == 1
    assert not os.path.exists(old)
    assert not os.listdir(cache)
