"""GGUF model files and their quantized tensors, for the MoE path: the ggml block table, ``QTensor`` (a matrix as its
raw blocks; ``dequantize`` on the GPU), ``dequant_rows`` / ``dequant_supported`` (the reference's ``_native`` entry
points, ``csrc/bindings/gguf.cpp:62-76``) and ``GGUFFile`` (the reference's reader API, ``src/artlite/gguf_model.py``
``GGUFFile.tensor`` / ``rows`` :494-525), which feeds ``moe.layer.MoELayer``.

The reader follows the GGUF file format (versions 2 and 3, little-endian): a header (magic ``GGUF``, u32 version, u64
tensor count, u64 key-value count), the key-values (a string key, a u32 value type, the value), the tensor infos (a
string name, u32 rank, u64 dims with the row length first, u32 ggml type, u64 offset into the data section), then
the data section at the next multiple of ``general.alignment`` (32 when absent). Strings are a u64 byte count and
UTF-8 bytes; arrays a u32 element type, a u64 count and the elements.

Dequantization runs in ``libartlite_moe`` for the types the reference's native dequantizer takes (F32, F16, BF16,
Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS), bit for bit the reference's fp32 values; other ggml types
are listed but not read (``NotImplementedError``)."""

import math
import mmap
from dataclasses import dataclass
from typing import NamedTuple

import numpy as np

from . import _hip

# ggml type id -> (name, values per block, bytes per block): the ggml format's table (the reference's _GGML_TYPES,
# gguf_model.py:385-390)
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 8: ("Q8_0", 32, 34),
              10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176),
              14: ("Q6_K", 256, 210), 16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98),
              19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82),
              23: ("IQ4_XS", 256, 136), 29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2)}
BLOCKS = {name: (per, nb) for name, per, nb in GGML_TYPES.values()}
TYPE_ID = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}
_PLAIN = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16}


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


class TensorInfo(NamedTuple):
    """A tensor of the file: dims (the row length first), ggml type name, absolute file offset, bytes (None for a
    type this build does not know the block size of)."""

    dims: tuple[int, ...]
    qtype: str
    offset: int
    nbytes: int | None


# GGUF value types: the fixed-size ones as numpy dtypes; 8 is a string, 9 an array
_FIXED = {0: np.dtype("<u1"), 1: np.dtype("<i1"), 2: np.dtype("<u2"), 3: np.dtype("<i2"), 4: np.dtype("<u4"),
          5: np.dtype("<i4"), 6: np.dtype("<f4"), 7: np.dtype("?"), 10: np.dtype("<u8"), 11: np.dtype("<i8"),
          12: np.dtype("<f8")}
_STR, _ARR = 8, 9


class _Cursor:
    """Reads the header's little-endian fields in order from the mapped bytes."""

    __slots__ = ("buf", "at")

    def __init__(self, buf: np.ndarray, at: int = 0):
        self.buf, self.at = buf, at

    def fixed(self, vtype: int, count: int = 1) -> np.ndarray:
        dt = _FIXED.get(vtype)
        if dt is None:
            raise ValueError(f"GGUF: unknown value type {vtype} at byte {self.at}")
        end = self.at + dt.itemsize * count
        if end > self.buf.size:
            raise ValueError("GGUF: the header runs past the end of the file")
        v = self.buf[self.at:end].view(dt)
        self.at = end
        return v

    def u32(self) -> int:
        return int(self.fixed(4)[0])

    def u64(self) -> int:
        return int(self.fixed(10)[0])

    def skip_string(self) -> tuple[int, int]:
        """(offset, length) of the string here, stepped over."""
        n = self.u64()
        start = self.at
        self.at += n
        if self.at > self.buf.size:
            raise ValueError("GGUF: a string runs past the end of the file")
        return start, n

    def string(self) -> str:
        start, n = self.skip_string()
        return self.buf[start:start + n].tobytes().decode("utf-8", errors="replace")

    def value(self, vtype: int) -> object:
        """One metadata value: Python scalars, str, numeric arrays as numpy arrays, string arrays as a
        ``StringArray`` (decoded on demand), nested arrays as lists."""
        if vtype == _STR:
            return self.string()
        if vtype != _ARR:
            return self.fixed(vtype)[0].item()
        etype, count = self.u32(), self.u64()
        if etype == _STR:
            first = self.at
            for _ in range(count):
                self.skip_string()
            return StringArray(self.buf, first, count)
        if etype == _ARR:
            return [self.value(_ARR) for _ in range(count)]
        return self.fixed(etype, count)


class StringArray:
    """A metadata array of strings (a vocabulary: hundreds of thousands), left in the mapped file until read."""

    def __init__(self, buf: np.ndarray, first: int, count: int):
        self._buf, self._first, self._count = buf, first, count

    def __len__(self) -> int:
        return self._count

    def __iter__(self):
        c = _Cursor(self._buf, self._first)
        for _ in range(self._count):
            yield c.string()

    def __getitem__(self, i: int) -> str:
        if not -self._count <= i < self._count:
            raise IndexError(i)
        c = _Cursor(self._buf, self._first)
        for _ in range(i % self._count):
            c.skip_string()
        return c.string()


class GGUFFile:
    """A GGUF file over a read-only memory map. ``meta``: key -> value; ``arch`` (``general.architecture``);
    ``tensor_info``: name -> ``TensorInfo``; ``tensor(name)`` a ``QTensor`` view of the mapped bytes (nothing is read
    until used); ``rows(name, idx)`` rows dequantized on the GPU."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            size = f.seek(0, 2)
            if size < 24:
                raise ValueError(f"{path}: not a GGUF file ({size} bytes)")
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self.data = np.frombuffer(self._map, np.uint8)
        try:
            self._parse()
        except ValueError as e:
            self.close()
            raise ValueError(f"{path}: {e}") from None

    def _parse(self) -> None:
        if self.data[:4].tobytes() != b"GGUF":
            raise ValueError("not a GGUF file")
        cur = _Cursor(self.data, 4)
        version = cur.u32()
        if version not in (2, 3):
            raise ValueError(f"GGUF version {version} (2 and 3 are read; a byte-swapped version is a big-endian file)")
        n_tensors, n_kv = cur.u64(), cur.u64()
        self.meta: dict[str, object] = {}
        for _ in range(n_kv):
            key = cur.string()
            self.meta[key] = cur.value(cur.u32())
        self.arch = str(self.meta.get("general.architecture", ""))
        entries = []
        for _ in range(n_tensors):
            name = cur.string()
            rank = cur.u32()
            dims = tuple(int(d) for d in cur.fixed(10, rank))
            entries.append((name, dims, cur.u32(), cur.u64()))
        align = int(self.meta.get("general.alignment", 32))
        if align <= 0:
            raise ValueError(f"alignment {align}")
        data_start = (cur.at + align - 1) // align * align
        self.tensor_info: dict[str, TensorInfo] = {}
        for name, dims, tid, rel in entries:
            qname, per, nb = GGML_TYPES.get(tid, (f"type{tid}", 1, None))
            n = math.prod(dims)
            nbytes = None if nb is None else n // per * nb
            if nbytes is not None and data_start + rel + nbytes > self.data.size:
                raise ValueError(f"tensor {name} ({nbytes} bytes at {data_start + rel}) runs past the end of the file")
            self.tensor_info[name] = TensorInfo(dims, qname, data_start + rel, nbytes)

    def close(self) -> None:
        """Release the mapping (views taken from it must not be used afterwards)."""
        self.data = np.empty(0, np.uint8)
        m, self._map = getattr(self, "_map", None), None
        if m is not None:
            try:
                m.close()
            except BufferError:  # (a view still refers to it: the mapping goes with the last view)
                pass

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def arch_meta(self, key: str, default: object = None) -> object:
        """Metadata value ``<architecture>.<key>``."""
        return self.meta.get(f"{self.arch}.{key}", default)

    def __contains__(self, name: str) -> bool:
        return name in self.tensor_info

    def tensor(self, name: str) -> QTensor:
        """The tensor as (rows, cols), its blocks along the columns; a vector is one row, a 3-D expert tensor
        (E experts of R rows) E R rows."""
        info = self.tensor_info[name]
        if info.nbytes is None:
            raise NotImplementedError(f"{name}: GGUF tensor type {info.qtype} is not supported")
        cols = info.dims[0]
        rows = math.prod(info.dims[1:])
        raw = self.data[info.offset:info.offset + info.nbytes]
        plain = _PLAIN.get(info.qtype)
        raw = raw.view(plain).reshape(rows, cols) if plain is not None else raw.reshape(rows, -1)
        return QTensor(name=name, qtype=info.qtype, rows=rows, cols=cols, raw=raw)

    def rows(self, name: str, idx: list[int] | np.ndarray, cols: int = 0, *, prefetch: bool = True) -> np.ndarray:
        """Rows ``idx`` of a tensor dequantized, (len(idx), cols) fp32, of their first ``cols`` columns (default all; a
        multiple of the format's block): the reference's ``GGUFFile.rows`` (gguf_model.py:508-525), dequantized on the
        GPU. prefetch: first ask the kernel for the rows' pages all at once (``madvise(MADV_WILLNEED)`` over each
        row's byte range), so that rows scattered over a file not yet in the page cache are read together rather than
        faulted in one by one."""
        t = self.tensor(name)
        cols, idx = cols or t.cols, np.asarray(idx, np.int64).reshape(-1)
        per, nb = BLOCKS[t.qtype]
        if cols % per or cols > t.cols:
            raise ValueError(f"{name}: {cols} columns of {t.cols} in blocks of {per}")
        if idx.size and (idx.min() < -t.rows or idx.max() >= t.rows):
            raise IndexError(f"{name}: row index out of range of {t.rows} rows")
        width = cols // per * nb  # (bytes of the leading columns)
        stride = t.raw.strides[0]
        if prefetch and idx.size > 1:
            self._willneed(self.tensor_info[name].offset + (idx % t.rows) * stride, width)
        raw = np.ascontiguousarray(t.raw.view(np.uint8).reshape(t.rows, -1)[idx, :width])
        out = np.empty((idx.size, cols), np.float32)
        dequant_rows(t.qtype, raw, out)
        return out

    def _willneed(self, starts: np.ndarray, nbytes: int) -> None:
        """madvise(MADV_WILLNEED) over the pages covering [start, start + nbytes) for each start (merged into runs)."""
        if self._map is None or not hasattr(mmap, "MADV_WILLNEED"):
            return
        page = mmap.PAGESIZE
        lo = np.unique(np.asarray(starts, np.int64) // page * page)
        hi = (lo + (nbytes + page - 1) // page * page + page).clip(max=len(self._map))
        run_lo, run_hi = int(lo[0]), int(hi[0])
        for a, b in zip(lo[1:].tolist(), hi[1:].tolist()):
            if a <= run_hi:
                run_hi = max(run_hi, b)
                continue
            self._map.madvise(mmap.MADV_WILLNEED, run_lo, run_hi - run_lo)
            run_lo, run_hi = a, b
        self._map.madvise(mmap.MADV_WILLNEED, run_lo, run_hi - run_lo)
