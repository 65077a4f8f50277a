"""The reference's C++ host step of an MoE layer, restated in numpy: the routing of tokens by their logits
(``artlite::moe_route``, ``csrc/artlite/moe_host.cpp:25-73,186-199``) and the plan of expert chunks dealt to the
columns (``artlite::moe_plan``, ``csrc/artlite/moe_host.cpp:201-235``), with the errors they raise.

Test infrastructure only (see ``oracle/__init__.py``)."""

import numpy as np

MIN_WEIGHT_SUM = 6.103515625e-5  # 2^-14 (``moe_host.cpp:41``)


class HostError(RuntimeError):
    """An argument error of the C++ host step (``artlite::Error`` in ``moe_host.cpp:188,207,223``)."""


def row_sum(e: np.ndarray) -> np.ndarray:
    """Per row of e (n, k) float64, the sum in numpy's pairwise order for k <= 128 (``moe_host.cpp:25-39``): below 8
    terms left to right from 0; else 8 running sums over strides of 8, combined as ((r0 + r1) + (r2 + r3)) + ((r4 + r5)
    + (r6 + r7)), then the remaining terms left to right."""
    n, k = e.shape
    if k < 8:
        s = np.zeros(n, np.float64)
        for j in range(k):
            s = s + e[:, j]
        return s
    assert k <= 128, k
    r = [e[:, j].copy() for j in range(8)]
    i = 8
    while i + 8 <= k:
        for j in range(8):
            r[j] = r[j] + e[:, i + j]
        i += 8
    s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
    for j in range(i, k):
        s = s + e[:, j]
    return s


def ordered_keys(lg: np.ndarray) -> np.ndarray:
    """The 32-bit ordered key of each fp32 logit (``moe_host.cpp:55``): the bits of l + 0 (so -0 is +0), negative
    values bit-inverted, non-negative ones with the sign bit set; unsigned order = float order."""
    u = (np.asarray(lg, np.float32) + np.float32(0.0)).view(np.uint32)
    return np.where(u >> np.uint32(31) != 0, ~u, u ^ np.uint32(0x80000000)).astype(np.uint32)


def gather_logits(logits: np.ndarray, n: int, row: int, per_col: int, pitch: int, E: int) -> np.ndarray:
    """The (n, E) logits of the router GEMM's layout (``moe_host.h:9-12``): expert e of token t at
    t row + (e / per_col) pitch + e % per_col of the flat array."""
    e = np.arange(E)
    idx = (np.arange(n)[:, None] * row) + (e // per_col) * pitch + e % per_col
    return np.asarray(logits, np.float32).reshape(-1)[idx]


def moe_route(logits: np.ndarray, n: int, row: int, per_col: int, pitch: int, E: int, k: int,
              sigmoid: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """``artlite::moe_route``: per token its k largest logits, largest first, ties to the lower id (the descending
    order of the 64-bit keys ordered-bits << 32 | ~id); weights e^(l - l0) in float64 over the k (softmax; l0 the
    largest) or sigmoid(l) (sigmoid), divided by their ``row_sum`` (sigmoid: at least 2^-14), rounded to float32.
    Returns (ids (n, k) int32, weights (n, k) float32)."""
    if k < 1 or k > E or per_col < 1 or E % per_col:
        raise HostError(f"moe_route: k {k} of E {E} ({per_col} per column)")
    lg = gather_logits(logits, n, row, per_col, pitch, E)
    key = ordered_keys(lg).astype(np.int64)
    ids = np.argsort(-key, axis=1, kind="stable")[:, :k].astype(np.int32)  # (stable: equal keys keep the lower id)
    top = np.take_along_axis(lg, ids, axis=1).astype(np.float64)
    if sigmoid:
        e = 1.0 / (1.0 + np.exp(-top))
        s = np.maximum(row_sum(e), MIN_WEIGHT_SUM)
    else:
        e = np.exp(top - top[:, :1])
        s = row_sum(e)
    return ids, (e / s[:, None]).astype(np.float32)


def moe_plan(ids: np.ndarray, E: int, cols: int, cap: int, chunk: int) -> dict[str, np.ndarray]:
    """``artlite::moe_plan``: the pairs p = t k + i by expert (a stable counting sort: histogram, exclusive prefix,
    scatter in p order), each expert's pairs in chunks of at most ``chunk``, the chunks dealt in turn to the
    ``cols`` columns (chunk j to column j % cols, its slot j // cols); rows of a chunk its tokens (padding: the first),
    pos[p] = (c cap + slot) chunk + row. Raises past ``cap`` chunks in a column or an id outside [0, E).
    Returns experts, counts, sizes, rows, pos (unused slots zero)."""
    ids = np.ascontiguousarray(ids, np.int32)
    n, k = ids.shape
    flat = ids.reshape(-1)
    bad = (flat < 0) | (flat >= E)
    if bad.any():
        raise HostError(f"moe_plan: expert id {int(flat[np.argmax(bad)])} of {E}")
    start = np.zeros(E + 1, np.int64)
    start[1:] = np.cumsum(np.bincount(flat, minlength=E))
    by = np.argsort(flat, kind="stable").astype(np.int64)  # (pairs by expert, in pair order)
    experts = np.zeros((cols, cap), np.int32)
    sizes = np.zeros((cols, cap), np.int32)
    rows = np.zeros((cols, cap, chunk), np.int32)
    pos = np.zeros((n, k), np.int64)
    counts = np.zeros(cols, np.int32)
    j = 0
    for x in range(E):
        for a in range(int(start[x]), int(start[x + 1]), chunk):
            b = min(a + chunk, int(start[x + 1]))
            c = j % cols
            kk = int(counts[c])
            if kk >= cap:
                raise HostError(f"moe_plan: more than {cap} chunks in a column")
            counts[c] += 1
            experts[c, kk] = x
            sizes[c, kk] = b - a
            toks = (by[a:b] // k).astype(np.int32)
            rows[c, kk, :b - a] = toks
            rows[c, kk, b - a:] = toks[0]
            pos.reshape(-1)[by[a:b]] = (c * cap + kk) * chunk + np.arange(b - a)
            j += 1
    return {"experts": experts, "counts": counts, "sizes": sizes, "rows": rows, "pos": pos}


def dispatch(ids: np.ndarray, E: int) -> dict[str, np.ndarray]:
    """The textbook stable counting sort under ``moe_plan`` (``moe_host.cpp:204-215``): counts (E,), offsets (E + 1,)
    exclusive prefix, order (P,) the pairs sorted by expert (pair order within an expert), slot (P,) each pair's
    position in that order."""
    flat = np.ascontiguousarray(ids, np.int64).reshape(-1)
    counts = np.bincount(flat, minlength=E).astype(np.int32)
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    slot = np.empty_like(order)
    slot[order] = np.arange(order.size, dtype=np.int32)
    return {"counts": counts, "offsets": offsets, "order": order, "slot": slot}
