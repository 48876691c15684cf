"""ctypes binding of ``libnhip.so``, the C ABI declared in ``include/nhip.h``.

Every call checks the int status and raises ``RuntimeError`` with ``nhip_last_error()``; the library must be
built (``__graft_entry__.build()`` or ``python -m lumen_amd.build``): there is no fallback.
"""

from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(_HERE, "libnhip.so")

_lib = None

NHIP_F32, NHIP_BF16, NHIP_F16 = 0, 1, 2
NHIP_BASE_WORKSPACE, NHIP_BASE_INPUT = 0, 1
NHIP_STEP_GEMM, NHIP_STEP_FLASH_FWD, NHIP_STEP_FLASH_BWD, NHIP_STEP_COPY, NHIP_STEP_FILL, NHIP_STEP_LCE = 1, 2, 3, 4, 5, 6
NHIP_LCE_I32, NHIP_LCE_I64 = 0, 1


class Props(C.Structure):
    _fields_ = [
        ("name", C.c_char * 64),
        ("arch", C.c_char * 32),
        ("compute_units", C.c_int32),
        ("xcds", C.c_int32),
        ("lds_bytes", C.c_int32),
        ("clock_khz", C.c_int32),
        ("memory_clock_khz", C.c_int32),
        ("memory_bus_bits", C.c_int32),
        ("l2_bytes", C.c_int32),
        ("hbm_bytes", C.c_size_t),
    ]


class GemmDesc(C.Structure):
    _fields_ = [
        ("m", C.c_int64),
        ("n", C.c_int64),
        ("k", C.c_int64),
        ("nbatch", C.c_int32),
        ("a_dtype", C.c_int32),
        ("b_dtype", C.c_int32),
        ("d_dtype", C.c_int32),
        ("batch", C.c_int64 * 3),
        ("a_batch", C.c_int64 * 3),
        ("b_batch", C.c_int64 * 3),
        ("d_batch", C.c_int64 * 3),
        ("a_m", C.c_int64),
        ("a_k", C.c_int64),
        ("b_k", C.c_int64),
        ("b_n", C.c_int64),
        ("d_m", C.c_int64),
        ("d_n", C.c_int64),
        ("config", C.c_int32),
        ("splits", C.c_int32),
    ]


class LceDesc(C.Structure):
    """``nhip_lce_desc``: linear cross entropy of h [b, d] and w [v, d] (include/nhip.h)."""

    _fields_ = [("b", C.c_int64), ("v", C.c_int64), ("d", C.c_int64), ("chunk_rows", C.c_int64),
                ("dtype", C.c_int32), ("target_dtype", C.c_int32)]


class AttnDesc(C.Structure):
    _fields_ = [
        ("batch", C.c_int64),
        ("heads", C.c_int64),
        ("kv_heads", C.c_int64),
        ("sq", C.c_int64),
        ("sk", C.c_int64),
        ("head_dim", C.c_int64),
        ("dtype", C.c_int32),
        ("causal", C.c_int32),
        ("scale", C.c_float),
        ("config", C.c_int32),
    ] + [(f"{t}_{a}", C.c_int64) for t in ("q", "k", "v", "o", "do", "dq", "dk", "dv") for a in ("b", "s", "n")] + [
        ("deterministic", C.c_int32),
        ("value_head_dim", C.c_int64),
    ]


class Reloc(C.Structure):
    _fields_ = [
        ("slot", C.c_uint32),
        ("base", C.c_uint32),
        ("index", C.c_uint32),
        ("pad", C.c_uint32),
        ("offset", C.c_uint64),
    ]


# Exported symbols and their argument types (the whole of include/nhip.h).
SIGNATURES = {
    "nhip_last_error": ([], C.c_char_p),
    "nhip_device_count": ([C.POINTER(C.c_int)], C.c_int),
    "nhip_set_device": ([C.c_int], C.c_int),
    "nhip_device_props": ([C.c_int, C.POINTER(Props)], C.c_int),
    "nhip_region_reserve": ([C.c_int, C.c_size_t], C.c_int),
    "nhip_alloc": ([C.c_int, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)], C.c_int),
    "nhip_free": ([C.c_int, C.c_void_p, C.c_size_t], C.c_int),
    "nhip_region_stats": ([C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)], C.c_int),
    "nhip_memcpy_h2d": ([C.c_void_p, C.c_void_p, C.c_size_t], C.c_int),
    "nhip_memcpy_d2h": ([C.c_void_p, C.c_void_p, C.c_size_t], C.c_int),
    "nhip_memcpy_d2d": ([C.c_void_p, C.c_void_p, C.c_size_t], C.c_int),
    "nhip_memset": ([C.c_void_p, C.c_int, C.c_size_t], C.c_int),
    "nhip_stream_sync": ([C.c_int], C.c_int),
    "nhip_event_create": ([C.POINTER(C.c_void_p)], C.c_int),
    "nhip_event_record": ([C.c_void_p], C.c_int),
    "nhip_event_elapsed_ms": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_float)], C.c_int),
    "nhip_event_destroy": ([C.c_void_p], C.c_int),
    "nhip_module_load": ([C.c_char_p, C.POINTER(C.c_void_p)], C.c_int),
    "nhip_module_function": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p)], C.c_int),
    "nhip_launch": (
        [C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_uint32, C.c_void_p, C.c_size_t],
        C.c_int,
    ),
    "nhip_gemm": ([C.POINTER(GemmDesc), C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "nhip_gemm_config_count": ([C.POINTER(C.c_int)], C.c_int),
    "nhip_gemm_splitk": ([C.POINTER(GemmDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "nhip_gemm_workspace": ([C.POINTER(GemmDesc), C.POINTER(C.c_size_t)], C.c_int),
    "nhip_linear_cross_entropy": ([C.POINTER(LceDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
                                  C.c_int),
    "nhip_linear_cross_entropy_workspace": ([C.POINTER(LceDesc), C.POINTER(C.c_size_t)], C.c_int),
    "nhip_flash_fwd": ([C.POINTER(AttnDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p], C.c_int),
    "nhip_flash_bwd": (
        [C.POINTER(AttnDesc)] + [C.c_void_p] * 10,
        C.c_int,
    ),
    "nhip_flash_bwd_workspace": ([C.POINTER(AttnDesc), C.POINTER(C.c_size_t)], C.c_int),
    "nhip_attn_config_count": ([C.POINTER(C.c_int)], C.c_int),
    "nhip_flash_bwd_noalloc": ([C.POINTER(AttnDesc)] + [C.c_void_p] * 9, C.c_int),
    "nhip_plan_create": ([C.POINTER(C.c_void_p)], C.c_int),
    "nhip_plan_destroy": ([C.c_void_p], C.c_int),
    "nhip_plan_add_launch": (
        [
            C.c_void_p,
            C.c_void_p,
            C.POINTER(C.c_uint32),
            C.POINTER(C.c_uint32),
            C.c_uint32,
            C.c_void_p,
            C.c_size_t,
            C.POINTER(Reloc),
            C.c_size_t,
        ],
        C.c_int,
    ),
    "nhip_plan_add_builtin": ([C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.POINTER(Reloc), C.c_size_t], C.c_int),
    "nhip_plan_run": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p), C.c_size_t], C.c_int),
    "nhip_plan_run_steps": (
        [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p), C.c_size_t, C.c_size_t, C.c_size_t],
        C.c_int,
    ),
    "nhip_plan_steps": ([C.c_void_p, C.POINTER(C.c_size_t)], C.c_int),
    "nhip_plan_profile": ([C.c_void_p, C.c_int], C.c_int),
    "nhip_plan_step_ms": ([C.c_void_p, C.POINTER(C.c_float), C.c_size_t], C.c_int),
    "nhip_plan_capture": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p), C.c_size_t, C.POINTER(C.c_void_p)], C.c_int),
    "nhip_graph_launch": ([C.c_void_p], C.c_int),
    "nhip_graph_destroy": ([C.c_void_p], C.c_int),
}


def lib():
    """The loaded library, its signatures set; RuntimeError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(
                f"{LIBRARY} is not built: the hip backend needs its native library (run __graft_entry__.build())"
            )
        lib_ = C.CDLL(LIBRARY)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(lib_, name)
            f.argtypes, f.restype = args, res
        _lib = lib_
    return _lib


def call(name, *args):
    """``name(*args)``, raising RuntimeError with the library's message on a nonzero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(lib().nhip_last_error().decode())
    return rc


def device_count():
    n = C.c_int(0)
    call("nhip_device_count", C.byref(n))
    return n.value


def set_device(device):
    call("nhip_set_device", device)


def props(device=0):
    p = Props()
    call("nhip_device_props", device, C.byref(p))
    return p


def alloc(device, nbytes, alignment=256):
    p = C.c_void_p()
    call("nhip_alloc", device, nbytes, alignment, C.byref(p))
    return p.value


def free(device, ptr, nbytes):
    call("nhip_free", device, ptr, nbytes)


def h2d(dst, src_ptr, nbytes):
    call("nhip_memcpy_h2d", dst, src_ptr, nbytes)


def d2h(dst_ptr, src, nbytes):
    call("nhip_memcpy_d2h", dst_ptr, src, nbytes)


def d2d(dst, src, nbytes):
    call("nhip_memcpy_d2d", dst, src, nbytes)


def sync(device=0):
    call("nhip_stream_sync", device)


class Event:
    """A HIP event on the device's stream (``lumen/runtime/event``)."""

    def __init__(self):
        self.handle = C.c_void_p()
        call("nhip_event_create", C.byref(self.handle))

    def record(self):
        call("nhip_event_record", self.handle)

    def elapsed_ms(self, end):
        ms = C.c_float()
        call("nhip_event_elapsed_ms", self.handle, end.handle, C.byref(ms))
        return ms.value

    def __del__(self):
        if _lib is not None and self.handle:
            _lib.nhip_event_destroy(self.handle)
            self.handle = None


def module_function(path, name):
    m = C.c_void_p()
    call("nhip_module_load", path.encode(), C.byref(m))
    f = C.c_void_p()
    call("nhip_module_function", m, name.encode(), C.byref(f))
    return f.value
