"""The GPU chunk plan (artlite_moe_plan) against the oracle's restatement of artlite::moe_plan, element for element,
and the reference's test_plan invariants (tests/moe/test_plan.py:36-67); its errors; multi-block dispatches."""

import numpy as np
import pytest

from artlite_amd import Error
from artlite_amd.moe import CHUNK, COLS
from artlite_amd.moe import plan as MP
from oracle import host_ref

pytestmark = pytest.mark.gpu


def _compare(ids: np.ndarray, E: int, cap: int) -> MP.Plan:
    plan = MP.Plan.of(ids, cap=cap, E=E)
    ref = host_ref.moe_plan(ids, E, COLS, cap, CHUNK)
    assert plan.counts == ref["counts"].tolist()
    for c in range(COLS):
        n = ref["counts"][c]
        assert np.array_equal(plan.experts[c], ref["experts"][c, :n])
        assert np.array_equal(plan.sizes[c], ref["sizes"][c, :n])
        assert np.array_equal(plan.rows[c], ref["rows"][c, :n])
    assert np.array_equal(plan.pos, ref["pos"])
    return plan


@pytest.mark.parametrize("T", [24, 2048])
def test_plan(T: int) -> None:
    """A routing's chunks: every pair once at its pos row of its expert's chunk, pairs in token order, ceil(r / CHUNK)
    chunks, columns within one chunk of each other, padding rows the chunk's first token."""
    rng = np.random.default_rng(T)
    ids, _ = MP.route(rng.standard_normal((T, 256)).astype(np.float32) + np.linspace(0, 3, 256, dtype=np.float32), 8)
    cap = -(-(256 + -(-T * 8 // CHUNK)) // COLS)
    plan = _compare(ids, 256, cap)
    counts = plan.counts
    assert max(counts) - min(counts) <= 1 and sum(counts) == sum(-(-r // CHUNK) for r in np.bincount(ids.ravel()))
    g, j = np.divmod(plan.pos, CHUNK)
    c, k = np.divmod(g, cap)
    assert len(set(plan.pos.ravel().tolist())) == ids.size
    for t in range(T):
        for i in range(8):
            assert plan.experts[c[t, i]][k[t, i]] == ids[t, i] and plan.rows[c[t, i]][k[t, i], j[t, i]] == t
    for col in range(COLS):
        for kk in range(counts[col]):
            r = plan.rows[col][kk]
            n = int(((c == col) & (k == kk)).sum())
            assert (r[n:] == r[0]).all() and (np.diff(r[:n]) > 0).all()


@pytest.mark.parametrize(("T", "k", "E"), [(4096, 8, 128), (3000, 6, 64), (1, 1, 1), (5000, 4, 1024)])
def test_plan_large_and_skewed(T: int, k: int, E: int) -> None:
    """Multi-block dispatches (up to 20000 pairs), skewed popularity, a single expert."""
    rng = np.random.default_rng(T + E)
    p = 1.0 / np.arange(1, E + 1) ** 1.2
    ids = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
    cap = -(-(E + -(-T * k // CHUNK)) // COLS)
    _compare(ids, E, cap)


def test_plan_errors() -> None:
    ids = np.array([[0, 1], [2, 7], [9, 1]], np.int32)
    with pytest.raises(Error, match="moe_plan: expert id 7 of 4"):
        MP.Plan.of(ids, cap=4, E=4)
    ids = np.zeros((1000, 1), np.int32)
    with pytest.raises(Error, match="more than 0 chunks in a column"):
        MP.Plan.of(ids, cap=0, E=4)
    plan = MP.Plan.of(np.zeros((0, 8), np.int32), cap=2, E=16)
    assert plan.counts == [0] * COLS and plan.pos.shape == (0, 8)
