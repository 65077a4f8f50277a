"""ctypes access to ``oracle/_ref/libartlite_ref.so``: the reference's own ``artlite::dequant_rows``
(``csrc/artlite/dequant.cpp:174-188``) compiled from its sources by ``oracle/Makefile``.

Test infrastructure only (see ``oracle/__init__.py``). ``available()`` is False where the library was not built (the
GPU box has no reference tree: the committed golden fixtures under ``tests/golden`` carry its outputs there)."""

import ctypes
from pathlib import Path

import numpy as np

PATH = Path(__file__).resolve().parent / "_ref" / "libartlite_ref.so"
_lib = None


def available() -> bool:
    return PATH.exists()


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(PATH))
        lib.ref_dequant_supported.argtypes = [ctypes.c_char_p]
        lib.ref_dequant_supported.restype = ctypes.c_int
        lib.ref_dequant_rows.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                         ctypes.c_size_t, ctypes.c_void_p]
        lib.ref_dequant_rows.restype = ctypes.c_int
        _lib = lib
    return _lib


def dequant_supported(qtype: str) -> bool:
    return bool(_load().ref_dequant_supported(qtype.encode()))


def dequant_rows(qtype: str, raw: np.ndarray, cols: int) -> np.ndarray:
    """The reference's fp32 rows of raw (n, row bytes) blocks."""
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty((raw.shape[0], cols), np.float32)
    rc = _load().ref_dequant_rows(qtype.encode(), raw.ctypes.data, raw.shape[0], raw.shape[1], cols, out.ctypes.data)
    if rc:
        raise RuntimeError(f"reference dequant_rows({qtype}) failed")
    return out
