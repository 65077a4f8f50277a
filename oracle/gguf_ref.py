"""GGUF quantized blocks in numpy: their exact fields and fp32 dequantization, restating
``src/artlite/gguf_model.py`` (``_f16`` :31-33, ``QTensor.fields`` :101-130, ``QTensor.dequantize`` :278-296, the
block table ``_GGML_TYPES`` :385-390) for the expert formats of this path: Q4_0, Q8_0, Q4_K (and the plain F32 / F16 /
BF16). The fp32 operations are the reference's, in its order, without fused multiply-adds.

Test infrastructure only (see ``oracle/__init__.py``)."""

import numpy as np

# ggml type id -> (name, values per block, bytes per block) (``gguf_model.py:385-390``)
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34), 12: ("Q4_K", 256, 144),
              30: ("BF16", 1, 2)}
BLOCKS = {name: (per, nb) for name, per, nb in GGML_TYPES.values()}
TYPE_ID = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}


def row_bytes(qtype: str, cols: int) -> int:
    """Bytes of a row of ``cols`` values."""
    per, nb = BLOCKS[qtype]
    assert cols % per == 0, (qtype, cols)
    return cols // per * nb


def f16_field(b: np.ndarray) -> np.ndarray:
    """(..., 2) uint8 little-endian fp16 -> (...) float32 (``gguf_model.py:31-33``; subnormals exact)."""
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float32)


def fields(qtype: str, raw: np.ndarray, cols: int) -> dict[str, np.ndarray]:
    """The exact fields of rows of blocks (``gguf_model.py:101-130``):
    Q4_0: d (rows, nb), q (rows, cols) u8 in [0, 15] (value j < 16 the low nibble of byte 2 + j, else the high nibble
    of byte 2 + j - 16);  Q8_0: d, q int8;  Q4_K: d, dmin (rows, nb), sc, mn (rows, nb, 8) u8 in [0, 63] (6-bit fields
    of the 12 scale bytes at 4), q u8 in [0, 15] (value l of group g: byte 16 + 32 (g // 2) + l, the low nibble for even
    g)."""
    raw = np.ascontiguousarray(raw, np.uint8)
    rows = raw.shape[0]
    per, nb = BLOCKS[qtype]
    b = raw.reshape(rows, cols // per, nb)
    if qtype == "Q4_0":
        q = np.empty((rows, b.shape[1], 32), np.uint8)
        q[..., :16] = b[..., 2:18] & 0xF
        q[..., 16:] = b[..., 2:18] >> 4
        return {"d": f16_field(b[..., 0:2]), "q": q.reshape(rows, cols)}
    if qtype == "Q8_0":
        return {"d": f16_field(b[..., 0:2]), "q": np.ascontiguousarray(b[..., 2:34]).view(np.int8).reshape(rows, cols)}
    if qtype == "Q4_K":
        lo, hi, top = b[..., 4:8], b[..., 8:12], b[..., 12:16]
        sc = np.concatenate([lo & 63, (top & 0xF) | ((lo >> 6) << 4)], axis=-1)
        mn = np.concatenate([hi & 63, (top >> 4) | ((hi >> 6) << 4)], axis=-1)
        qs = b[..., 16:144].reshape(rows, -1, 4, 32)
        q = np.stack([qs & 0xF, qs >> 4], axis=3)  # (rows, nb, chunk, half, 32): group g = 2 chunk + half
        return {"d": f16_field(b[..., 0:2]), "dmin": f16_field(b[..., 2:4]), "sc": sc, "mn": mn,
                "q": q.reshape(rows, cols)}
    raise ValueError(qtype)


def dequantize(qtype: str, raw: np.ndarray, cols: int) -> np.ndarray:
    """fp32 (rows, cols) weights (``gguf_model.py:278-296``): Q4_0 d (q - 8); Q8_0 d q; Q4_K (d sc) q - dmin mn, each
    product and the difference rounded to fp32 on its own; F32 / F16 / BF16 their values."""
    raw = np.ascontiguousarray(raw)
    rows = raw.shape[0]
    if qtype == "F32":
        return raw.view(np.float32).reshape(rows, -1)[:, :cols].astype(np.float32)
    if qtype == "F16":
        return raw.view(np.float16).reshape(rows, -1)[:, :cols].astype(np.float32)
    if qtype == "BF16":
        u = raw.view(np.uint16).reshape(rows, -1)[:, :cols].astype(np.uint32) << np.uint32(16)
        return u.view(np.float32)
    f = fields(qtype, raw, cols)
    with np.errstate(invalid="ignore", over="ignore"):  # (infinite fp16 scales: inf * 0 is NaN, as in C++)
        if qtype == "Q4_0":
            w = f["d"][..., None] * (f["q"].reshape(rows, -1, 32).astype(np.float32) - np.float32(8.0))
        elif qtype == "Q8_0":
            w = f["d"][..., None] * f["q"].reshape(rows, -1, 32).astype(np.float32)
        elif qtype == "Q4_K":
            a = f["d"][..., None] * f["sc"].astype(np.float32)
            m = f["dmin"][..., None] * f["mn"].astype(np.float32)
            w = a[..., None] * f["q"].reshape(rows, -1, 8, 32).astype(np.float32) - m[..., None]
        else:
            raise ValueError(qtype)
    return np.ascontiguousarray(w, dtype=np.float32).reshape(rows, cols)
