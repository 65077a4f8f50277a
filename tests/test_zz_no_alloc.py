"""``artlite_moe_plan_static`` (the chunk plan that allocates nothing: its device memory one static array per GPU)
through the C ABI against ``artlite_moe_plan`` on the same ids: every output array bit for bit, on two calls in a row
(the second smaller, so stale contents of the shared array would show), with bad ids, and its size limit."""

import ctypes

import numpy as np
import pytest

from artlite_amd import _hip
from artlite_amd.moe import CHUNK, COLS

pytestmark = pytest.mark.gpu


def _plan(fn: str, ids: np.ndarray, E: int, cap: int) -> tuple[int, list[np.ndarray]]:
    """(status, [experts, counts, sizes, rows, pos]) of one call, the outputs pre-filled with a pattern (entries a
    call does not deal keep it, as with the reference's arrays)."""
    out = [np.full((COLS, cap), -7, np.int32), np.full(COLS, -7, np.int32), np.full((COLS, cap), -7, np.int32),
           np.full((COLS, cap, CHUNK), -7, np.int32), np.full(ids.shape, -7, np.int64)]
    c = ctypes
    rc = getattr(_hip.lib(), fn)(_hip.ptr(ids, c.c_int32), ids.shape[0], ids.shape[1], E, COLS, cap, CHUNK,
                                 _hip.ptr(out[0], c.c_int32), _hip.ptr(out[1], c.c_int32), _hip.ptr(out[2], c.c_int32),
                                 _hip.ptr(out[3], c.c_int32), _hip.ptr(out[4], c.c_int64))
    return rc, out


def _ids(T: int, k: int, E: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    return np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)


def test_plan_static_matches_plan() -> None:
    for T, k, E in ((4096, 8, 128), (300, 6, 64), (4096, 8, 128), (1, 1, 1)):  # (large, smaller, large again, tiny)
        ids = _ids(T, k, E, T + E)
        cap = -(-(E + -(-T * k // CHUNK)) // COLS)
        rc0, want = _plan("artlite_moe_plan", ids, E, cap)
        rc1, got = _plan("artlite_moe_plan_static", ids, E, cap)
        assert rc0 == rc1 == _hip.OK, _hip.last_error()
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)


def test_plan_static_errors() -> None:
    ids = np.array([[0, 1], [2, 9], [3, 1]], np.int32)
    rc, _ = _plan("artlite_moe_plan_static", ids, 4, 4)
    assert rc == _hip.EINVAL and _hip.last_error() == "moe_plan: expert id 9 of 4"
    ok = np.array([[0, 1], [2, 3]], np.int32)  # (after the error: the counters start from zero again)
    rc0, want = _plan("artlite_moe_plan", ok, 4, 4)
    rc1, got = _plan("artlite_moe_plan_static", ok, 4, 4)
    assert rc0 == rc1 == _hip.OK
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)
    big = np.zeros((400_000, 1), np.int32)
    rc, _ = _plan("artlite_moe_plan_static", big, 8, 2200)
    assert rc == _hip.EINVAL and "bytes of device scratch" in _hip.last_error()


def _free_bytes() -> int:
    """The device's free memory (hipMemGetInfo of the HIP runtime this process has loaded)."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_plan_static_allocates_nothing() -> None:
    """After a first call (the array's address resolved), calls of growing size within the limit leave the device's
    free memory as it was; artlite_moe_plan on a larger batch than it has seen grows its buffers (the contrast)."""
    E, k = 128, 8
    ids0 = _ids(64, k, E, 1)
    cap0 = -(-(E + -(-64 * k // CHUNK)) // COLS)
    assert _plan("artlite_moe_plan_static", ids0, E, cap0)[0] == _hip.OK
    before = _free_bytes()
    for T in (256, 1024, 8192, 20000):
        ids = _ids(T, k, E, T)
        cap = -(-(E + -(-T * k // CHUNK)) // COLS)
        assert _plan("artlite_moe_plan_static", ids, E, cap)[0] == _hip.OK, _hip.last_error()
        assert _free_bytes() == before, T
    T = 1 << 20  # (8 M pairs: tens of MB of staged ids, histograms and results)
    ids = np.random.default_rng(0).integers(0, E, (T, k), dtype=np.int32)
    cap = -(-(E + -(-T * k // CHUNK)) // COLS)
    assert _plan("artlite_moe_plan", ids, E, cap)[0] == _hip.OK, _hip.last_error()
    assert _free_bytes() < before
