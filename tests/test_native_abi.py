"""The C ABI: libnhip.so loads on a machine without a GPU and exports every function include/nhip.h
declares; the ctypes binding names exactly those functions."""

import ctypes as C
import os
import re

from lumen_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "nhip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(nhip_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(native.LIBRARY)
    names = _declared()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name


def test_binding_covers_the_header():
    assert sorted(native.SIGNATURES) == _declared()


def test_device_count_without_a_gpu_is_an_answer():
    """nhip_device_count succeeds (0 devices where there is no GPU, as in the build container)."""
    n = native.device_count()
    assert n >= 0
