"""GPU routing (``artlite_moe_route``, ``artlite_moe_top_k``) against the oracle: the known answers of the reference's
routing tests (tests/moe/test_route.py:16-26, tests/moe/test_plan.py:18-33), the decode ``route.route`` (GPU top k
then the deal), ids bit-exact against the C++ host routing's restatement over many E / k shapes, NaN logits, sigmoid
gating, no tokens."""

import numpy as np
import pytest

from artlite_amd.moe import COLS
from artlite_amd.moe import plan as MP
from artlite_amd.moe import route as MR
from oracle import host_ref, moe_ref

from . import known_answers
from .helpers import ulp_diff

pytestmark = pytest.mark.gpu


def test_top_k() -> None:
    """The decode cores' top 8 on the planted rows (equal maxima in id order, an all-equal row) and 61 random ones:
    the layer oracle's ids; its weights within 2e-6; the weights are the float64 softmax of the chosen logits."""
    lg, planted = known_answers.planted_logits(64)
    ids, w = MR.top_k(lg, 8)
    known_answers.assert_planted(ids, {r: planted[r] for r in (0, 1)})
    want_ids, want_w = moe_ref.moe_route(lg, 8)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_allclose(w, want_w, rtol=0, atol=2e-6)
    chosen = np.take_along_axis(lg, ids, 1).astype(np.float64)
    soft = np.exp(chosen - chosen[:, :1])
    np.testing.assert_allclose(w, soft / soft.sum(1, keepdims=True), rtol=0, atol=1e-15)


def test_route() -> None:
    """1024 tokens with the planted rows (equal maxima, all equal, +0 / -0), as plain rows and in the router GEMM's
    layout (NaN gaps never read): the layer oracle's ids, weights within 2e-7."""
    lg, planted = known_answers.planted_logits(1024)
    want_ids, want_w = moe_ref.moe_route(lg, 8)
    known_answers.assert_planted(want_ids, planted)
    for ids, w in (MP.route(lg, 8), MP.route(known_answers.router_gemm_rows(lg), 8, E=256, per_col=32, pitch=64)):
        np.testing.assert_array_equal(ids, want_ids)
        np.testing.assert_allclose(w, want_w, rtol=0, atol=2e-7)


def test_decode_route() -> None:
    """``route.route``: the GPU top k, then the deal of every chosen expert over the columns; against the layer
    oracle's ids and the deal invariants, and the per-item weights against a per-slot lookup."""
    for S, E, k in ((4, 256, 8), (3, 128, 8), (1, 64, 6), (5, 96, 4)):  # (unions of at most 32: the deal's range)
        lg = (np.random.default_rng(S * E + k).standard_normal((S, E)) * 1.5).astype(np.float32)
        ids, w, items = MR.route(lg, k, COLS)
        want_ids, want_w = moe_ref.moe_route(lg, k)
        np.testing.assert_array_equal(ids, want_ids)
        np.testing.assert_allclose(w, want_w, rtol=0, atol=2e-6)
        union = sorted(set(ids.ravel().tolist()))
        known_answers.check_deal(items, union, COLS, MR.MAX_ITEMS)
        for e in union:
            per_slot = [float(w[s, list(ids[s]).index(e)]) if e in ids[s] else 0.0 for s in range(S)]
            assert MR.item_weights(ids, w, e).tolist() == per_slot
    ids, w, items = MR.route(lg, k, COLS, gating="sigmoid")
    hids, hw = host_ref.moe_route(lg.reshape(-1), lg.shape[0], E, E, 0, E, k, sigmoid=True)
    np.testing.assert_array_equal(ids, hids)
    np.testing.assert_allclose(w, hw, rtol=2e-7, atol=0)


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
