"""The C ABI (include/artlite_moe.h) without a GPU: the library loads, exports every declared function, rejects bad
arguments with the reference's messages before touching a device, and fails loudly (no CPU fallback) when a compute
call finds no GPU. Plus the host-only parts of the operator API (the decode deal, item weights) against the
reference's test_deal (tests/moe/test_route.py:29-41)."""

import re
from pathlib import Path

import numpy as np
import pytest

from artlite_amd import _hip
from artlite_amd.moe import COLS
from artlite_amd.moe import route as MR

from . import known_answers

HEADER = Path(__file__).resolve().parents[1] / "include" / "artlite_moe.h"


def declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(artlite_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_bound_api() -> None:
    """The header's functions are exactly the ones the ctypes binding declares."""
    assert declared() == sorted(_hip.SIGNATURES)


def test_library_exports_every_symbol() -> None:
    lib = _hip.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.artlite_version()


def test_argument_errors_before_any_device() -> None:
    """moe_route's k / E / per_col check (moe_host.cpp:188) and its "arrays too small" (bindings/moe.cpp:25-28)."""
    lg = np.zeros((2, 8), np.float32)
    with pytest.raises(_hip.Error, match=r"moe_route: k 9 of E 8 \(8 per column\)"):
        from artlite_amd.moe import plan

        plan.route(lg, 9)
    c = _hip.ctypes
    ids, w = np.zeros(16, np.int32), np.zeros(16, np.float32)
    rc = _hip.lib().artlite_moe_route(_hip.ptr(lg.reshape(-1), c.c_float), 3, 2, 8, 8, 0, 8, 2, 0,
                                      _hip.ptr(ids, c.c_int32), _hip.ptr(w, c.c_float))
    assert rc == _hip.EINVAL and _hip.last_error() == "moe_route: arrays too small"
    rc = _hip.lib().artlite_dequant_rows(b"Q4_0", None, 1, 10, 32, None)
    assert rc == _hip.EINVAL and "32 columns of rows of 10 B" in _hip.last_error()
    assert _hip.lib().artlite_dequant_supported(b"Q4_K") and not _hip.lib().artlite_dequant_supported(b"Q5_0")


@pytest.mark.skipif(_hip.LIB_PATH.exists() and _hip.device_count() > 0, reason="a GPU is visible")
def test_no_gpu_fails_loudly() -> None:
    """Without a GPU a valid compute call raises (there is no CPU fallback)."""
    from artlite_amd.moe import plan

    with pytest.raises(_hip.Error, match="no HIP device"):
        plan.route(np.zeros((2, 8), np.float32), 2)


@pytest.mark.parametrize("u", [0, 1, 8, 13, 17, 21, 31, 32])
def test_deal(u: int) -> None:
    """Unions of u chosen experts (the reference test_deal's sizes, plus 0 and 1) dealt over the 8 columns: the deal
    invariants."""
    union = np.sort(np.random.default_rng(u).permutation(256)[:u]).tolist()
    known_answers.check_deal(MR.deal(union, COLS), union, COLS, MR.MAX_ITEMS)


def test_item_weights() -> None:
    ids = np.array([[3, 5], [5, 7]])
    w = np.array([[0.75, 0.25], [0.5, 0.5]])
    assert MR.item_weights(ids, w, 5).tolist() == [0.25, 0.5]
    assert MR.item_weights(ids, w, 9).tolist() == [0.0, 0.0]


def test_layer_shape_limits_before_any_device() -> None:
    """A layer whose products the MFMA decode tiles cannot stage (K beyond 4096) is refused at create."""
    from artlite_amd.moe.layer import MoELayer

    for H, F, sF in ((8192, 512, 0), (1024, 6144, 0), (1024, 512, 8192)):
        with pytest.raises(_hip.Error, match="at most 4096 each"):
            MoELayer(hidden=H, n_experts=8, top_k=2, expert_ffn=F, gate_type="Q4_0", down_type="Q4_0", max_tokens=4,
                     shared_ffn=sF, shared_type="Q4_0" if sF else "")
