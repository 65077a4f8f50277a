"""A minimal GGUF (v3) writer for tests: metadata values and raw tensors, laid out as the format specifies (header,
key-values, tensor infos, data at the alignment). Test infrastructure only.

Metadata values: str; bool; int (int32, or int64 beyond it); float (float32); a list / array of ints (int32), of
floats (float64) or of strs; or an explicit ``(value type code, value)`` pair for any scalar type (0 u8 .. 12 f64)."""

import struct

import numpy as np

_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(v: object) -> bytes:
    """The value type code and bytes of one metadata value."""
    if isinstance(v, tuple):
        code, x = v
        return struct.pack("<I", code) + struct.pack(_FMT[code], x)
    if isinstance(v, str):
        return struct.pack("<I", 8) + _string(v)
    if isinstance(v, bool):
        return struct.pack("<I?", 7, v)
    if isinstance(v, int):
        code = 5 if -2 ** 31 <= v < 2 ** 31 else 11
        return struct.pack("<I", code) + struct.pack(_FMT[code], v)
    if isinstance(v, float):
        return struct.pack("<If", 6, v)
    items = list(v)
    if items and isinstance(items[0], str):
        return struct.pack("<IIQ", 9, 8, len(items)) + b"".join(_string(s) for s in items)
    a = np.asarray(items)
    if a.dtype.kind == "f":
        return struct.pack("<IIQ", 9, 12, a.size) + a.astype("<f8").tobytes()
    return struct.pack("<IIQ", 9, 5, a.size) + a.astype("<i4").tobytes()


def write_gguf(path: str, meta: dict, tensors: list[tuple[str, tuple[int, ...], int, np.ndarray]],
               alignment: int = 32) -> None:
    """tensors: (name, dims (GGUF order: the row length first), ggml type id, raw bytes or values)."""
    kv = b"".join(_string(key) + _value(v) for key, v in meta.items())
    infos, data, off = b"", b"", 0
    for name, dims, ttype, raw in tensors:
        blob = np.ascontiguousarray(raw).tobytes()
        infos += _string(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        infos += struct.pack("<IQ", ttype, off)
        pad = -len(blob) % alignment
        data += blob + b"\0" * pad
        off += len(blob) + pad
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)) + kv + infos
    head += b"\0" * (-len(head) % alignment)
    with open(path, "wb") as f:
        f.write(head + data)
