"""GGUF model files and their quantized tensors (the reference's ``src/artlite/gguf_model.py`` for this path):
the ggml block table, ``QTensor`` (raw blocks, ``dequantize`` on the GPU), ``dequant_rows`` / ``dequant_supported``
(the reference's ``_native`` entry points), and ``GGUFFile``, a reader of the file's memory map (metadata, tensor
infos, ``tensor``, ``rows``) that feeds ``moe.layer.MoELayer.upload``.

Dequantization runs in ``libartlite_moe`` for the types the reference's native dequantizer takes (F32, F16, BF16,
Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS), bit for bit the reference's fp32 values; other ggml types
are listed but not read (``NotImplementedError``, as the reference does for unknown types)."""

import math
import struct
from dataclasses import dataclass

import numpy as np

from . import _hip

# ggml type id -> (name, values per block, bytes per block) (the reference's _GGML_TYPES, gguf_model.py:385-390)
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 8: ("Q8_0", 32, 34),
              10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176),
              14: ("Q6_K", 256, 210), 16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98),
              19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82),
              23: ("IQ4_XS", 256, 136), 29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2)}
BLOCKS = {name: (per, nb) for name, per, nb in GGML_TYPES.values()}
TYPE_ID = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}


def dequant_supported(qtype: str) -> bool:
    """Whether ``dequant_rows`` reads a GGUF type on the GPU (``artlite_dequant_supported``)."""
    return bool(_hip.lib().artlite_dequant_supported(qtype.encode()))


def dequant_rows(qtype: str, raw: np.ndarray, out: np.ndarray) -> None:
    """GGUF rows (raw: (n, row bytes) uint8) dequantized into out (n, cols) fp32, its first cols columns
    (``artlite_dequant_rows``; the reference's ``_native.dequant_rows``, csrc/bindings/gguf.cpp:62-73)."""
    raw = np.ascontiguousarray(raw, np.uint8)
    if out.shape[0] != raw.shape[0]:
        raise _hip.Error("dequant_rows: out's rows are not raw's")
    assert out.dtype == np.float32 and out.flags.c_contiguous
    c = _hip.ctypes
    _hip.check(_hip.lib().artlite_dequant_rows(qtype.encode(), _hip.ptr(raw, c.c_uint8), raw.shape[0],
                                               raw.shape[1] if raw.ndim == 2 else 0, out.shape[1],
                                               _hip.ptr(out, c.c_float)))


@dataclass
class QTensor:
    """One weight matrix (rows = output features, cols = K) as its raw GGUF bytes (rows, row bytes)."""

    name: str
    qtype: str
    rows: int
    cols: int
    raw: np.ndarray

    @property
    def row_bytes(self) -> int:
        per, nb = BLOCKS[self.qtype]
        return self.cols // per * nb

    def dequantize(self) -> np.ndarray:
        """fp32 (rows, cols) weights, computed on the GPU (the reference's ``QTensor.dequantize`` values)."""
        if not dequant_supported(self.qtype):
            raise NotImplementedError(f"{self.name}: {self.qtype} is not read by this build")
        out = np.empty((self.rows, self.cols), np.float32)
        dequant_rows(self.qtype, np.ascontiguousarray(self.raw).view(np.uint8).reshape(self.rows, -1), out)
        return out


# GGUF metadata value types: scalar struct formats (8: string, 9: array)
_KV_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_KV_STRING, _KV_ARRAY = 8, 9


class GGUFFile:
    """A GGUF file read from its memory map: ``meta`` (scalars, strings, numeric arrays; string arrays are skipped),
    ``tensor_info`` (name -> (dims, type name, file offset, bytes or None for unknown types)), ``tensor(name)``."""

    def __init__(self, path: str):
        self.path = path
        self.data = np.memmap(path, dtype=np.uint8, mode="r")
        buf = memoryview(self.data)
        if bytes(buf[:4]) != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        version, n_tensors, n_kv = struct.unpack_from("<IQQ", buf, 4)
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {version}")
        pos = 24

        def string(p: int) -> tuple[str, int]:
            n = int.from_bytes(buf[p:p + 8], "little")
            return bytes(buf[p + 8:p + 8 + n]).decode("utf-8", errors="replace"), p + 8 + n

        self.meta: dict[str, object] = {}
        for _ in range(n_kv):
            key, pos = string(pos)
            (vt,) = struct.unpack_from("<I", buf, pos)
            pos += 4
            if vt == _KV_STRING:
                self.meta[key], pos = string(pos)
            elif vt == _KV_ARRAY:
                et, count = struct.unpack_from("<IQ", buf, pos)
                pos += 12
                if et == _KV_STRING:
                    for _ in range(count):
                        pos += 8 + int.from_bytes(buf[pos:pos + 8], "little")
                else:
                    dt = np.dtype(_KV_SCALAR[et])
                    self.meta[key] = np.frombuffer(buf, dt, count, pos)
                    pos += count * dt.itemsize
            else:
                fmt = _KV_SCALAR[vt]
                (self.meta[key],) = struct.unpack_from(fmt, buf, pos)
                pos += struct.calcsize(fmt)
        infos = []
        for _ in range(n_tensors):
            name, pos = string(pos)
            (nd,) = struct.unpack_from("<I", buf, pos)
            dims = struct.unpack_from(f"<{nd}Q", buf, pos + 4)
            ttype, off = struct.unpack_from("<IQ", buf, pos + 4 + 8 * nd)
            pos += 16 + 8 * nd
            infos.append((name, dims, ttype, off))
        align = int(self.meta.get("general.alignment", 32))
        base = -(-pos // align) * align
        self.arch = str(self.meta.get("general.architecture", ""))
        self.tensor_info: dict[str, tuple[tuple[int, ...], str, int, int | None]] = {}
        for name, dims, ttype, off in infos:
            tname, per, nb = GGML_TYPES.get(ttype, (f"type{ttype}", 1, None))
            n = math.prod(dims)
            self.tensor_info[name] = (dims, tname, base + off, None if nb is None else n // per * nb)

    def arch_meta(self, key: str, default: object = None) -> object:
        return self.meta.get(f"{self.arch}.{key}", default)

    def __contains__(self, name: str) -> bool:
        return name in self.tensor_info

    def tensor(self, name: str) -> QTensor:
        """The tensor as (rows, cols), blocks along the columns (a 3-D expert tensor: E x rows-per-expert rows)."""
        dims, qtype, off, nbytes = self.tensor_info[name]
        if nbytes is None:
            raise NotImplementedError(f"{name}: GGUF tensor type {qtype} is not supported")
        cols = dims[0]
        rows = math.prod(dims[1:]) if len(dims) > 1 else 1
        raw = self.data[off:off + nbytes]
        if qtype in ("F32", "F16", "BF16"):
            raw = raw.view({"F32": np.float32, "F16": np.float16, "BF16": np.uint16}[qtype]).reshape(rows, cols)
        else:
            raw = raw.reshape(rows, -1)
        return QTensor(name=name, qtype=qtype, rows=rows, cols=cols, raw=raw)

    def rows(self, name: str, idx: list[int] | np.ndarray, cols: int = 0) -> np.ndarray:
        """Rows ``idx`` of a tensor dequantized (len(idx), cols) fp32, of its first ``cols`` columns (default all):
        the reference's ``GGUFFile.rows`` (gguf_model.py:508-525), on the GPU."""
        t = self.tensor(name)
        cols, idx = cols or t.cols, np.asarray(idx)
        per, nb = BLOCKS[t.qtype]
        width = cols // per * nb if per > 1 else cols
        raw = np.ascontiguousarray(t.raw[idx, :width]).view(np.uint8)
        out = np.empty((len(idx), cols), np.float32)
        dequant_rows(t.qtype, raw.reshape(len(idx), -1), out)
        return out
