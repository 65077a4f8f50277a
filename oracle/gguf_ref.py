"""GGUF quantized blocks in numpy: their exact fields and fp32 dequantization, restating
``src/artlite/gguf_model.py`` (``_f16`` :31-33, ``QTensor.fields`` :101-163,195-206, ``QTensor.dequantize`` :278-331,
``IQ4_VALUES`` :370-371, the block table ``_GGML_TYPES`` :385-390) for the types the reference's native dequantizer
takes (``csrc/artlite/dequant.cpp:145-150``): Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS and the plain
F32 / F16 / BF16. The fp32 operations are the reference's, in its order, without fused multiply-adds.

Test infrastructure only (see ``oracle/__init__.py``)."""

import numpy as np

# ggml type id -> (name, values per block, bytes per block) (``gguf_model.py:385-390``)
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 8: ("Q8_0", 32, 34),
              11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
              20: ("IQ4_NL", 32, 18), 23: ("IQ4_XS", 256, 136), 30: ("BF16", 1, 2)}
BLOCKS = {name: (per, nb) for name, per, nb in GGML_TYPES.values()}
TYPE_ID = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}
# IQ4_NL / IQ4_XS's 16 values (ggml's kvalues_iq4nl; ``gguf_model.py:370-371``)
IQ4_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int8)


def row_bytes(qtype: str, cols: int) -> int:
    """Bytes of a row of ``cols`` values."""
    per, nb = BLOCKS[qtype]
    assert cols % per == 0, (qtype, cols)
    return cols // per * nb


def f16_field(b: np.ndarray) -> np.ndarray:
    """(..., 2) uint8 little-endian fp16 -> (...) float32 (``gguf_model.py:31-33``; subnormals exact)."""
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float32)


def _nibbles32(b: np.ndarray) -> np.ndarray:
    """(..., 16) code bytes of 32-value groups -> (..., 32) u8 codes in Q4_0's order: value j < 16 the low nibble of
    byte j, value 16 + j its high nibble."""
    return np.concatenate([b & 0xF, b >> 4], axis=-1)


def _k_scales(s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Q4_K / Q5_K's 12 scale bytes (..., 12) -> the 8 groups' 6-bit scales and mins (..., 8) u8."""
    lo, hi, top = s[..., 0:4], s[..., 4:8], s[..., 8:12]
    return (np.concatenate([lo & 63, (top & 0xF) | ((lo >> 6) << 4)], axis=-1),
            np.concatenate([hi & 63, (top >> 4) | ((hi >> 6) << 4)], axis=-1))


def fields(qtype: str, raw: np.ndarray, cols: int) -> dict[str, np.ndarray]:
    """The exact fields of rows of blocks (``gguf_model.py:101-163,195-206``), codes as (rows, cols) arrays in value
    order and scales per block or sub-block:
    Q4_0 / IQ4_NL: d (rows, nb), q u8 [0, 15] (value j < 16 the low nibble of byte 2 + j, else the high nibble of byte
    2 + j - 16); Q4_1: d, m, q as Q4_0's from byte 4;  Q8_0: d, q int8;
    Q4_K / Q5_K: d, dmin (rows, nb), sc, mn (rows, nb, 8) u8 [0, 63] (6-bit fields of the 12 scale bytes at 4), q u8
    (value l of group g: byte 16 (Q5_K: 48) + 32 (g // 2) + l, the low nibble for even g; Q5_K: bit g of qh[l], the 32
    bytes at 16, is bit 4 of the code);
    Q6_K: d (at 208), sc (rows, nb, 16) int8 (at 192), q u8 [0, 63] (value 128 h + 32 jj + l: the low (jj < 2) or high
    nibble of ql[64 h + 32 (jj % 2) + l], bits 4..5 crumb jj of qh[32 h + l], qh at 128);
    Q3_K: d (at 108), sc (rows, nb, 16) int8 = the 6-bit scale - 32 (low nibbles of bytes 96..103 for sub-blocks 0..7,
    their high nibbles for 8..15, the top crumb of sub-block 4 k + i in bits 2 k of byte 104 + i), q u8 [0, 7] (value
    128 n + 32 j + 16 h + l: crumb j of qs[32 n + 16 h + l] at 32, bit 2 from bit 4 n + j of hmask[16 h + l]);
    IQ4_XS: d (rows, nb), ls (rows, nb, 8) u8 [0, 63] (nibble g % 2 of byte 4 + g // 2, bits 4..5 crumb g of the u16 at
    2), q u8 [0, 15] (a group's 16 bytes at 8 + 16 g in Q4_0's order)."""
    raw = np.ascontiguousarray(raw, np.uint8)
    rows = raw.shape[0]
    per, nb = BLOCKS[qtype]
    b = raw.reshape(rows, cols // per, nb)
    n = b.shape[1]
    if qtype in ("Q4_0", "IQ4_NL"):
        return {"d": f16_field(b[..., 0:2]), "q": _nibbles32(b[..., 2:18]).reshape(rows, cols)}
    if qtype == "Q4_1":
        return {"d": f16_field(b[..., 0:2]), "m": f16_field(b[..., 2:4]), "q": _nibbles32(b[..., 4:20]).reshape(rows, cols)}
    if qtype == "Q8_0":
        return {"d": f16_field(b[..., 0:2]), "q": np.ascontiguousarray(b[..., 2:34]).view(np.int8).reshape(rows, cols)}
    if qtype in ("Q4_K", "Q5_K"):
        sc, mn = _k_scales(b[..., 4:16])
        qs = b[..., (16 if qtype == "Q4_K" else 48):].reshape(rows, n, 4, 32)
        q = np.stack([qs & 0xF, qs >> 4], axis=3).reshape(rows, n, 8, 32)  # group g = 2 chunk + half
        if qtype == "Q5_K":
            qh = b[..., 16:48]  # (rows, n, 32)
            q = q | (((qh[..., None, :] >> np.arange(8, dtype=np.uint8)[:, None]) & 1) << 4)
        return {"d": f16_field(b[..., 0:2]), "dmin": f16_field(b[..., 2:4]), "sc": sc, "mn": mn,
                "q": q.reshape(rows, cols)}
    if qtype == "Q6_K":
        ql = b[..., 0:128].reshape(rows, n, 2, 2, 32)  # (h, jj % 2, l)
        qh = b[..., 128:192].reshape(rows, n, 2, 1, 32)
        lo = np.stack([ql[..., 0, :] & 0xF, ql[..., 1, :] & 0xF, ql[..., 0, :] >> 4, ql[..., 1, :] >> 4], axis=3)
        jj = np.arange(4, dtype=np.uint8)[:, None]
        q = lo | (((qh >> (2 * jj)) & 3) << 4)  # (rows, n, h, jj, l)
        return {"d": f16_field(b[..., 208:210]), "sc": np.ascontiguousarray(b[..., 192:208]).view(np.int8),
                "q": q.reshape(rows, cols)}
    if qtype == "Q3_K":
        j = np.arange(4, dtype=np.uint8).reshape(1, 1, 1, 4, 1, 1)
        nn = np.arange(2, dtype=np.uint8).reshape(1, 1, 2, 1, 1, 1)
        qs = b[..., 32:96].reshape(rows, n, 2, 1, 2, 16)  # (n, -, h, l)
        hm = b[..., 0:32].reshape(rows, n, 1, 1, 2, 16)
        q = ((qs >> (2 * j)) & 3) | (((hm >> (4 * nn + j)) & 1) << 2)  # (rows, n, nn, j, h, l)
        s = b[..., 96:108]
        lo = np.concatenate([s[..., :8] & 0xF, s[..., :8] >> 4], axis=-1)
        hi = (s[..., 8:12, None] >> (2 * np.arange(4, dtype=np.uint8))) & 3  # (rows, n, i, k): sub-block 4 k + i
        sc6 = lo | (hi.transpose(0, 1, 3, 2).reshape(rows, n, 16) << 4)
        return {"d": f16_field(b[..., 108:110]), "sc": (sc6.astype(np.int16) - 32).astype(np.int8),
                "q": q.reshape(rows, cols)}
    if qtype == "IQ4_XS":
        sh = np.ascontiguousarray(b[..., 2:4]).view("<u2")  # (rows, n, 1)
        g = np.arange(8)
        ls = ((b[..., 4 + g // 2] >> (4 * (g & 1)).astype(np.uint8)) & 15) | \
            (((sh >> (2 * g).astype(np.uint16)) & 3).astype(np.uint8) << 4)
        q = _nibbles32(b[..., 8:136].reshape(rows, n, 8, 16))
        return {"d": f16_field(b[..., 0:2]), "ls": ls, "q": q.reshape(rows, cols)}
    raise ValueError(qtype)


def dequantize(qtype: str, raw: np.ndarray, cols: int) -> np.ndarray:
    """fp32 (rows, cols) weights (``gguf_model.py:278-331``): Q4_0 d (q - 8); Q4_1 d q + m; Q8_0 d q; Q4_K / Q5_K
    (d sc) q - dmin mn; Q6_K (d sc) (q - 32); Q3_K (d sc) (q - 4); IQ4_NL d IQ4[q]; IQ4_XS (d (ls - 32)) IQ4[q]; each
    product, sum and difference rounded to fp32 on its own; F32 / F16 / BF16 their values."""
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
        elif qtype == "Q4_1":
            w = f["d"][..., None] * f["q"].reshape(rows, -1, 32).astype(np.float32) + f["m"][..., None]
        elif qtype == "Q8_0":
            w = f["d"][..., None] * f["q"].reshape(rows, -1, 32).astype(np.float32)
        elif qtype in ("Q4_K", "Q5_K"):
            a = f["d"][..., None] * f["sc"].astype(np.float32)
            m = f["dmin"][..., None] * f["mn"].astype(np.float32)
            w = a[..., None] * f["q"].reshape(rows, -1, 8, 32).astype(np.float32) - m[..., None]
        elif qtype in ("Q6_K", "Q3_K"):
            a = f["d"][..., None] * f["sc"].astype(np.float32)  # (rows, nb, 16)
            off = np.float32(32.0 if qtype == "Q6_K" else 4.0)
            w = a[..., None] * (f["q"].reshape(rows, -1, 16, 16).astype(np.float32) - off)
        elif qtype == "IQ4_NL":
            w = f["d"][..., None] * IQ4_VALUES[f["q"]].reshape(rows, -1, 32).astype(np.float32)
        elif qtype == "IQ4_XS":
            dl = f["d"][..., None] * (f["ls"].astype(np.float32) - np.float32(32.0))  # (rows, nb, 8)
            w = dl[..., None] * IQ4_VALUES[f["q"]].reshape(rows, -1, 8, 32).astype(np.float32)
        else:
            raise ValueError(qtype)
    return np.ascontiguousarray(w, dtype=np.float32).reshape(rows, cols)
