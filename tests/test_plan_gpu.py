"""The GPU chunk plan (``artlite_moe_plan``) element for element against the oracle's restatement of
``artlite::moe_plan``, plus the plan invariants of the reference's test_plan (tests/moe/test_plan.py:36-67), for the
reference's routings, multi-block dispatches and skewed popularity; its argument errors."""

import numpy as np
import pytest

from artlite_amd import Error
from artlite_amd.moe import CHUNK, COLS
from artlite_amd.moe import plan as MP
from oracle import host_ref

from . import known_answers

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
    """The reference test_plan's routings (experts biased by a ramp, top 8 of 256): the oracle's plan element for
    element, and the plan invariants."""
    rng = np.random.default_rng(T)
    ramp = np.linspace(0, 3, 256, dtype=np.float32)
    ids, _ = MP.route(rng.standard_normal((T, 256)).astype(np.float32) + ramp, 8)
    cap = -(-(256 + -(-T * 8 // CHUNK)) // COLS)
    known_answers.check_plan(_compare(ids, 256, cap), ids, cap)


@pytest.mark.parametrize(("T", "k", "E"), [(4096, 8, 128), (3000, 6, 64), (1, 1, 1), (5000, 4, 1024)])
def test_plan_large_and_skewed(T: int, k: int, E: int) -> None:
    """Multi-block dispatches (up to 20000 pairs), skewed popularity, a single expert."""
    rng = np.random.default_rng(T + E)
    p = 1.0 / np.arange(1, E + 1) ** 1.2
    ids = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
    cap = -(-(E + -(-T * k // CHUNK)) // COLS)
    known_answers.check_plan(_compare(ids, E, cap), ids, cap)


def test_plan_errors() -> None:
    ids = np.array([[0, 1], [2, 7], [9, 1]], np.int32)
    with pytest.raises(Error, match="moe_plan: expert id 7 of 4"):
        MP.Plan.of(ids, cap=4, E=4)
    ids = np.zeros((1000, 1), np.int32)
    with pytest.raises(Error, match="more than 0 chunks in a column"):
        MP.Plan.of(ids, cap=0, E=4)
    plan = MP.Plan.of(np.zeros((0, 8), np.int32), cap=2, E=16)
    assert plan.counts == [0] * COLS and plan.pos.shape == (0, 8)
