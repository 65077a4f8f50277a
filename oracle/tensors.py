"""Seeded random GGUF blocks and bf16 helpers, torch-free.

``random_blocks`` restates ``random_tensor`` of ``tests/tensors.py:15-41`` for the block types of this path: every
byte uniform, then the fp16 fields at the type's offsets (``BLOCK``, ``tests/tensors.py:9-12``) overwritten with
N(0, scale) values (``abs_scales``: their magnitudes, as the benchmark configurations ask).

Test infrastructure only (see ``oracle/__init__.py``)."""

import numpy as np

from .gguf_ref import BLOCKS

# the offsets of each block type's fp16 fields (``tests/tensors.py:9-12``)
F16_OFFSETS = {"Q4_0": (0,), "Q4_1": (0, 2), "Q8_0": (0,), "Q3_K": (108,), "Q4_K": (0, 2), "Q5_K": (0, 2),
               "Q6_K": (208,), "IQ4_NL": (0,), "IQ4_XS": (0,)}


def random_blocks(qtype: str, rows: int, cols: int, seed: int | np.random.Generator, *, scale: float = 0.01,
                  abs_scales: bool = False) -> np.ndarray:
    """(rows, row bytes) uint8 of random ``qtype`` blocks: bytes uniform in [0, 256), the fp16 fields N(0, scale)
    (``abs_scales``: |N(0, scale)|) in the order of ``tests/tensors.py:33-37``."""
    rng = seed if isinstance(seed, np.random.Generator) else np.random.default_rng(seed)
    per, nb = BLOCKS[qtype]
    n = cols // per
    raw = rng.integers(0, 256, (rows, n, nb), dtype=np.uint8)
    for o in F16_OFFSETS[qtype]:
        d = rng.standard_normal((rows, n)) * scale
        d = (np.abs(d) if abs_scales else d).astype(np.float16)
        raw[..., o:o + 2] = d.view(np.uint8).reshape(rows, n, 2)
    return raw.reshape(rows, n * nb)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), rounded to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 (exact)."""
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 rounded to the nearest bf16 value, as fp32."""
    return from_bf16_bits(bf16_bits(x))
