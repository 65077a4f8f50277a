"""ctypes binding of ``libartlite_moe.so`` (the C ABI of ``include/artlite_moe.h``): argument types, status codes to
``Error``. No torch: arrays cross as numpy buffers.

The library is loaded on first use. There is no CPU fallback: without the built library, or without a GPU, every
compute call raises ``Error``."""

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libartlite_moe.so"

OK, EINVAL, EHIP, ENOMEM = 0, 1, 2, 3


class Error(RuntimeError):
    """An error of the MoE library: the reference's ``_native.Error`` (``csrc/bindings/errors.cpp:19``), which derives
    from RuntimeError too."""


c_i32p = ctypes.POINTER(ctypes.c_int32)
c_i64p = ctypes.POINTER(ctypes.c_int64)
c_f32p = ctypes.POINTER(ctypes.c_float)
c_f64p = ctypes.POINTER(ctypes.c_double)
c_u8p = ctypes.POINTER(ctypes.c_uint8)


class Desc(ctypes.Structure):
    """``artlite_moe_desc``."""

    _fields_ = [(name, ctypes.c_int32) for name in (
        "hidden", "n_experts", "top_k", "expert_ffn", "gate_type", "down_type", "shared_ffn", "shared_type",
        "shared_gated", "gating", "max_tokens")] + [("norm_eps", ctypes.c_float), ("residual", ctypes.c_int32),
                                                    ("shared_down_type", ctypes.c_int32)]


# every exported function: (restype, argtypes)
SIGNATURES = {
    "artlite_last_error": (ctypes.c_size_t, [ctypes.c_char_p, ctypes.c_size_t]),
    "artlite_version": (ctypes.c_char_p, []),
    "artlite_device_count": (ctypes.c_int, [c_i32p]),
    "artlite_moe_route": (ctypes.c_int, [c_f32p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_i32p, c_f32p]),
    "artlite_moe_top_k": (ctypes.c_int, [c_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, c_i32p,
                                         c_f64p]),
    "artlite_moe_plan": (ctypes.c_int, [c_i32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, c_i32p, c_i32p, c_i32p, c_i32p, c_i64p]),
    "artlite_moe_plan_static": (ctypes.c_int, [c_i32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, c_i32p, c_i32p, c_i32p, c_i32p, c_i64p]),
    "artlite_dequant_supported": (ctypes.c_int, [ctypes.c_char_p]),
    "artlite_dequant_rows": (ctypes.c_int, [ctypes.c_char_p, c_u8p, ctypes.c_size_t, ctypes.c_size_t,
                                            ctypes.c_size_t, c_f32p]),
    "artlite_moe_layer_create": (ctypes.c_int, [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_void_p)]),
    "artlite_moe_layer_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "artlite_moe_layer_upload": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]),
    "artlite_moe_layer_forward": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                                 c_f32p]),
    "artlite_moe_layer_stage": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64]),
    "artlite_moe_layer_run": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64]),
    "artlite_moe_layer_sync": (ctypes.c_int, [ctypes.c_void_p]),
    "artlite_moe_layer_output": (ctypes.c_int, [ctypes.c_void_p, c_f32p, ctypes.c_int64]),
    "artlite_moe_layer_tap": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]),
    "artlite_moe_layer_time": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.c_int64,
                                              ctypes.c_int, ctypes.c_int, c_f64p, c_f64p, c_f64p, ctypes.c_int,
                                              c_i32p]),
    "artlite_moe_kernel_names": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_char_p, ctypes.c_size_t]),
    "artlite_hbm_copy": (ctypes.c_int, [ctypes.c_size_t, ctypes.c_int, c_f64p]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises ``Error`` when it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise Error(f"{LIB_PATH} is not built: python -m artlite_amd.build (the HIP library is required; there is "
                        "no CPU fallback)")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(h, name)
            f.restype, f.argtypes = res, args
        _lib = h
    return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().artlite_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int) -> None:
    """Raise ``Error`` with the library's message for a non-zero status."""
    if rc != OK:
        raise Error(last_error())


def ptr(a: np.ndarray, ctype: type) -> object:
    """A C pointer to a C-contiguous array's data."""
    assert a.flags.c_contiguous, "arrays crossing the C ABI are C-contiguous"
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def device_count() -> int:
    n = ctypes.c_int32(0)
    check(lib().artlite_device_count(ctypes.byref(n)))
    return n.value
