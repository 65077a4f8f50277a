"""A minimal GGUF (v3) writer for tests: metadata scalars / strings / numeric arrays and raw tensors, laid out as the
format specifies (header, key-values, tensor infos, data at the alignment). Test infrastructure only."""

import struct

import numpy as np

_SCALAR = {int: (5, "<i"), float: (6, "<f"), bool: (7, "<?")}


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path: str, meta: dict, tensors: list[tuple[str, tuple[int, ...], int, np.ndarray]],
               alignment: int = 32) -> None:
    """tensors: (name, dims (GGUF order: the row length first), ggml type id, raw bytes or values)."""
    kv = b""
    for key, v in meta.items():
        kv += _string(key)
        if isinstance(v, str):
            kv += struct.pack("<I", 8) + _string(v)
        elif isinstance(v, (list, np.ndarray)) and not isinstance(v, str):
            a = np.asarray(v, np.int32)
            kv += struct.pack("<IIQ", 9, 5, a.size) + a.tobytes()
        else:
            vt, fmt = _SCALAR[type(v)]
            kv += struct.pack("<I", vt) + struct.pack(fmt, v)
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
