"""GPU routing (artlite_moe_route / artlite_moe_top_k) against the oracle: the reference's test_top_k
(tests/moe/test_route.py:16-26) and test_route (tests/moe/test_plan.py:18-33), bit-exact ids against the C++ host
routing's restatement for every supported E / k shape, NaN logits, sigmoid gating, the empty case."""

import numpy as np
import pytest

from artlite_amd.moe import COLS
from artlite_amd.moe import plan as MP
from artlite_amd.moe import route as MR
from oracle import host_ref, moe_ref

from .helpers import ulp_diff

pytestmark = pytest.mark.gpu


def test_top_k() -> None:
    """The cores' top 8 (ties to the lower id) and weights against moe_ref.moe_route, ties included."""
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((64, 256)).astype(np.float32) * 2
    lg[0, [3, 9, 200]] = lg[0].max() + 1
    lg[1, :] = 0.5
    ids, w = MR.top_k(lg, 8)
    rids, rw = moe_ref.moe_route(lg, 8)
    assert np.array_equal(ids, rids)
    assert np.abs(w - rw).max() < 2e-6
    assert ids[0, :3].tolist() == [3, 9, 200] and ids[1].tolist() == list(range(8))
    e = np.exp(np.take_along_axis(lg, ids, 1).astype(np.float64) - lg.max(1, keepdims=True))
    assert np.abs(w - e / e.sum(1, keepdims=True)).max() < 1e-15


def test_route() -> None:
    """The reference's test_route: both layouts, 1024 tokens; the oracle's ids, weights within 2e-7."""
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((1024, 256)).astype(np.float32) * 2
    lg[0, [3, 9, 200]] = lg[0].max() + 1
    lg[1, :] = 0.5
    lg[2, :8], lg[2, 8:] = -0.0, -1
    lg[2, 5] = 0.0
    rids, rw = moe_ref.moe_route(lg, 8)
    rows = np.full((1024, COLS, 64), np.nan, np.float32)
    rows[:, :, :32] = lg.reshape(1024, COLS, 32)
    for ids, w in (MP.route(lg, 8), MP.route(rows.reshape(1024, -1), 8, E=256, per_col=32, pitch=64)):
        assert np.array_equal(ids, rids)
        assert np.abs(w - rw).max() < 2e-7
    assert rids[0, :3].tolist() == [3, 9, 200] and rids[1].tolist() == rids[2].tolist() == list(range(8))


@pytest.mark.parametrize(("E", "k"), [(8, 2), (60, 4), (64, 6), (65, 1), (128, 8), (256, 8), (256, 16), (512, 8),
                                      (1000, 12), (1024, 64)])
def test_route_shapes(E: int, k: int) -> None:
    """Bit-exact ids against the C++ host routing's restatement; weights within one float32 ulp of it (numpy's and
    the GPU's float64 exp may differ in the last double bit)."""
    rng = np.random.default_rng(E * 100 + k)
    T = 300
    lg = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
    lg[::7] = np.round(lg[::7])  # (ties)
    ids, w = MP.route(lg, k)
    hids, hw = host_ref.moe_route(lg.reshape(-1), T, E, E, 0, E, k)
    assert np.array_equal(ids, hids)
    assert ulp_diff(w, hw).max() <= 1 and (w == hw).mean() > 0.99


def test_route_sigmoid_and_nan() -> None:
    """Sigmoid gating against the restatement; a NaN logit ranks by its bits as in the C++ keys."""
    rng = np.random.default_rng(9)
    lg = rng.standard_normal((200, 128)).astype(np.float32) * 3
    lg[5, 17] = np.nan
    lg[6, 3] = -np.float32(np.nan)
    lg[7] = -40.0
    ids, w = MP.route(lg, 8, gating="sigmoid")
    hids, hw = host_ref.moe_route(lg.reshape(-1), 200, 128, 128, 0, 128, 8, sigmoid=True)
    assert np.array_equal(ids, hids)
    ok = ~np.isnan(hw)
    assert np.array_equal(np.isnan(w), ~ok) and ulp_diff(w[ok], hw[ok]).max() <= 1
    assert ids[5, 0] == 17


def test_route_empty_and_errors() -> None:
    ids, w = MP.route(np.zeros((0, 16), np.float32), 4)
    assert ids.shape == (0, 4) and w.shape == (0, 4)
    from artlite_amd import Error

    with pytest.raises(Error, match=r"k 3 of E 6 \(4 per column\)"):
        MP.route(np.zeros((2, 8), np.float32), 3, E=6, per_col=4, pitch=4)
