"""Writes ``tests/golden/dequant_golden.npz``: GGUF blocks and their fp32 values as computed by the reference's own
C++ dequantizer (``csrc/artlite/dequant.cpp``, compiled from its sources into ``oracle/_ref`` by ``oracle/Makefile``).

Per quantized type the reference's native dequantizer takes (Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL,
IQ4_XS): 8 rows of seeded random blocks (the reference's ``random_tensor`` recipe) and 8 rows of edge blocks (extreme
codes, subnormal / negative / zero / largest / infinite fp16 scales, sub-block scales and mins at their extremes:
6-bit 0 and 63, int8 -128, -1 and 127).
Run from the repository root: ``python tests/golden/make_golden.py`` (needs ``make -C oracle`` first)."""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref_lib  # noqa: E402
from oracle.gguf_ref import BLOCKS  # noqa: E402
from oracle.tensors import F16_OFFSETS, random_blocks  # noqa: E402

QTYPES = ("Q4_0", "Q4_1", "Q8_0", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS")

COLS = 512
F16 = {"one": 0x3C00, "sub": 0x0001, "sub_max": 0x03FF, "neg_half": 0xB800, "zero": 0x0000, "neg_zero": 0x8000,
       "max": 0x7BFF, "min_normal": 0x0400, "inf": 0x7C00}


def _set_f16(raw: np.ndarray, row: int, nb: int, off: int, bits: int) -> None:
    b = raw[row].reshape(-1, nb)
    b[:, off] = bits & 0xFF
    b[:, off + 1] = bits >> 8


def edge_rows(qtype: str) -> np.ndarray:
    per, nb = BLOCKS[qtype]
    n = COLS // per
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 256, (8, n * nb), dtype=np.uint8)
    if qtype in ("Q4_0", "Q8_0"):
        fill = [0x00, 0xFF, 0x80, 0x7F, 0x81, None, None, None]
        scales = ["one", "one", "sub", "neg_half", "sub_max", "neg_zero", "max", "inf"]
        for r in range(8):
            b = raw[r].reshape(n, nb)
            if fill[r] is not None:
                b[:, 2:] = fill[r]
            _set_f16(raw, r, nb, 0, F16[scales[r]])
    elif qtype != "Q4_K":
        # every byte but the fp16 fields one value (codes, high bits, sub-block scales and mins: 0x00 -> codes 0 and
        # 6-bit scales 0, 0xFF -> the largest codes and 6-bit scales 63 (int8 -1), 0x80 / 0x7F -> int8 -128 / 127),
        # or random; the fp16 fields at their edges
        fill = [0x00, 0xFF, 0x80, 0x7F, 0x55, None, None, None]
        first = ["one", "one", "sub", "neg_half", "sub_max", "neg_zero", "max", "inf"]
        second = ["one", "sub", "one", "min_normal", "neg_zero", "one", "sub_max", "one"]
        offs = F16_OFFSETS[qtype]
        for r in range(8):
            b = raw[r].reshape(n, nb)
            if fill[r] is not None:
                b[:] = fill[r]
            for o, name in zip(offs, (first[r], second[r])):
                _set_f16(raw, r, nb, o, F16[name])
    else:  # Q4_K
        specs = [("one", "one", 0xFF, 0x00), ("one", "sub", 0xFF, 0xFF), ("sub", "one", 0x00, 0x5A),
                 ("neg_half", "min_normal", None, None), ("zero", "neg_zero", None, None), ("max", "one", 0x11, 0x77),
                 ("sub_max", "sub_max", 0xFF, None), ("inf", "one", None, None)]
        for r, (d, dmin, sc, q) in enumerate(specs):
            b = raw[r].reshape(n, nb)
            _set_f16(raw, r, nb, 0, F16[d])
            _set_f16(raw, r, nb, 2, F16[dmin])
            if sc is not None:
                b[:, 4:16] = sc
            if q is not None:
                b[:, 16:] = q
    return raw


def main() -> None:
    if not ref_lib.available():
        raise SystemExit("oracle/_ref/libartlite_ref.so is not built: make -C oracle")
    out = {}
    for qtype in QTYPES:
        rnd = random_blocks(qtype, 8, COLS, 1, scale=0.01)
        raw = np.concatenate([rnd, edge_rows(qtype)])
        out[f"raw_{qtype}"] = raw
        out[f"out_{qtype}"] = ref_lib.dequant_rows(qtype, raw, COLS).view(np.uint32)
    path = Path(__file__).resolve().parent / "dequant_golden.npz"
    np.savez_compressed(path, cols=np.array(COLS), **out)
    print(path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
