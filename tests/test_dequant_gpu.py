"""GPU dequantization (artlite_dequant_rows) bit for bit against the reference's own outputs (tests/golden, made by
its compiled dequant.cpp) and the oracle: the reference's test_dequant_rows (tests/test_gguf_model.py:116-124)."""

from pathlib import Path

import numpy as np
import pytest

from artlite_amd import Error, gguf_model
from oracle import gguf_ref, tensors

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "dequant_golden.npz"


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


QTYPES = ("Q4_0", "Q4_1", "Q8_0", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS")


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_golden(qtype: str) -> None:
    z = np.load(GOLDEN)
    cols = int(z["cols"])
    raw = z[f"raw_{qtype}"]
    out = np.empty((raw.shape[0], cols), np.float32)
    gguf_model.dequant_rows(qtype, raw, out)
    assert _same_bits(out, z[f"out_{qtype}"].view(np.float32))


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_rows(qtype: str) -> None:
    """The reference's test: 33 x 1024 random blocks (seed 1), bit-identical; and a row subset of fewer columns."""
    raw = tensors.random_blocks(qtype, 33, 1024, 1)
    t = gguf_model.QTensor("t", qtype, 33, 1024, raw)
    assert _same_bits(t.dequantize(), gguf_ref.dequantize(qtype, raw, 1024))
    out = np.empty((33, 512), np.float32)
    gguf_model.dequant_rows(qtype, raw, out)
    assert _same_bits(out, gguf_ref.dequantize(qtype, raw, 1024)[:, :512])


def test_dequant_plain_types() -> None:
    rng = np.random.default_rng(2)
    v = (rng.standard_normal((5, 64)) * 3).astype(np.float32)
    for qtype, raw in (("F32", v.view(np.uint8)), ("F16", v.astype(np.float16).view(np.uint8)),
                       ("BF16", tensors.bf16_bits(v).view(np.uint8))):
        out = np.empty((5, 64), np.float32)
        gguf_model.dequant_rows(qtype, raw.reshape(5, -1), out)
        assert _same_bits(out, gguf_ref.dequantize(qtype, raw.reshape(5, -1), 64))


def test_dequant_errors() -> None:
    assert all(gguf_model.dequant_supported(q) for q in QTYPES + ("F32", "F16", "BF16"))
    assert not gguf_model.dequant_supported("IQ2_XS") and not gguf_model.dequant_supported("Q2_K")
    with pytest.raises(Error, match="no native Q2_K"):
        gguf_model.dequant_rows("Q2_K", np.zeros((1, 84), np.uint8), np.empty((1, 256), np.float32))
    with pytest.raises(Error, match="64 columns of rows of 18 B"):
        gguf_model.dequant_rows("Q4_0", np.zeros((1, 18), np.uint8), np.empty((1, 64), np.float32))
