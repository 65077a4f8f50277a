"""Known-answer inputs and invariant checks shared by the oracle's and the GPU's routing / plan / deal tests.

The planted rows are the reference tests' known answers (``tests/moe/test_route.py:16-26``,
``tests/moe/test_plan.py:18-33``): a three-way tie for the largest logit must come out in id order, a row of equal
logits must pick the lowest ids, and +0 / -0 must tie. The checks restate the invariants of the reference's
``test_plan`` (``tests/moe/test_plan.py:36-67``) and ``test_deal`` (``tests/moe/test_route.py:29-41``)."""

from collections import Counter

import numpy as np

from artlite_amd.moe import CHUNK, COLS


def planted_logits(T: int, E: int = 256, seed: int = 0) -> tuple[np.ndarray, dict[int, list[int]]]:
    """N(0, 4) fp32 logits (T, E), E > 200, T >= 3, with rows 0..2 planted; returns (logits, {row: the ids its top 8
    must start with})."""
    lg = (np.random.default_rng(seed).standard_normal((T, E)) * 2).astype(np.float32)
    top = np.float32(lg[0].max() + 1)
    lg[0, [200, 3, 9]] = top                 # three equal maxima, planted out of order
    lg[1] = np.float32(0.5)                  # nothing to choose between: ids 0..7
    lg[2] = np.float32(-1.0)
    lg[2, :8] = np.float32(-0.0)             # eight zeros of both signs on top
    lg[2, 5] = np.float32(0.0)
    return lg, {0: [3, 9, 200], 1: list(range(8)), 2: list(range(8))}


def assert_planted(ids: np.ndarray, planted: dict[int, list[int]]) -> None:
    for row, lead in planted.items():
        assert ids[row, :len(lead)].tolist() == lead, (row, ids[row].tolist())


def router_gemm_rows(lg: np.ndarray, per_col: int = 32, pitch: int = 64) -> np.ndarray:
    """The same logits in the router GEMM's row layout: COLS groups of per_col experts, each at a pitch of ``pitch``
    floats, NaN in the gaps (which routing must never read)."""
    T, E = lg.shape
    assert E == COLS * per_col
    rows = np.full((T, COLS, pitch), np.nan, np.float32)
    rows[:, :, :per_col] = lg.reshape(T, COLS, per_col)
    return rows.reshape(T, -1)


def check_plan(plan, ids: np.ndarray, cap: int) -> None:
    """A chunk plan of routing ids (T, k) (``experts`` / ``sizes`` / ``rows`` per column, ``pos``): each pair at its
    own row, in a chunk of its expert, the chunk's row list naming its token; chunk sizes the pairs placed there; the
    pairs of a chunk in token order, padding repeating the chunk's first token; ceil(pairs / CHUNK) chunks per expert
    in total; columns within one chunk of each other."""
    T, k = ids.shape
    n = np.array(plan.counts)
    assert n.max() - n.min() <= 1
    assert n.sum() == (-(-np.bincount(ids.ravel()) // CHUNK)).sum()
    ex = np.full((COLS, cap), -1, np.int64)
    size = np.zeros((COLS, cap), np.int64)
    rows = np.full((COLS, cap, CHUNK), -1, np.int64)
    for col in range(COLS):
        ex[col, :n[col]], size[col, :n[col]], rows[col, :n[col]] = plan.experts[col], plan.sizes[col], plan.rows[col]
    pos = np.asarray(plan.pos)
    assert pos.shape == ids.shape and np.unique(pos).size == ids.size
    chunk, j = np.divmod(pos, CHUNK)
    col, slot = np.divmod(chunk, cap)
    assert (ex[col, slot] == ids).all()
    assert (rows[col, slot, j] == np.arange(T)[:, None]).all()
    placed = np.zeros((COLS, cap), np.int64)
    np.add.at(placed, (col, slot), 1)
    assert (placed == size).all()
    for c in range(COLS):
        for s in range(n[c]):
            r, m = rows[c, s], size[c, s]
            assert (np.diff(r[:m]) > 0).all() and (r[m:] == r[0]).all(), (c, s)


def check_deal(items: list, union: list[int], cols: int, max_items: int) -> None:
    """A deal of the union's experts over ``cols`` columns: each half of each expert exactly once; per column whole
    experts before halves, at most ``max_items`` items; the busiest column ceil(2 |union| / cols) halves."""
    got = Counter((e, h) for col in items for e, h0, h1 in col for h in range(h0, h1 + 1))
    assert got == Counter((e, h) for e in union for h in (0, 1))
    assert max(map(len, items)) <= max_items
    load = [sum(h1 - h0 + 1 for _, h0, h1 in col) for col in items]
    assert max(load) == -(-2 * len(union) // cols)
    for col in items:
        spans = [h1 - h0 for _, h0, h1 in col]
        assert spans == sorted(spans, reverse=True)
