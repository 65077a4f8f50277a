"""The MoE FFN layer oracle in float32 numpy (restating ``tests/moe/ref.py``, llama.cpp's ``build_moe_ffn``).

Test infrastructure only (see ``oracle/__init__.py``)."""

from collections.abc import Callable

import numpy as np

from .np_ops import f32, sigmoid, silu, softmax

MIN_WEIGHT_SUM = np.float32(6.103515625e-5)  # 2^-14, the clamp of the weights' sum (``tests/moe/ref.py:18``)


def moe_route(logits: np.ndarray, k: int, gating: str = "softmax") -> tuple[np.ndarray, np.ndarray]:
    """The router's choice (``tests/moe/ref.py:11-18``): p = softmax(logits) (or sigmoid), the k largest p per token
    (a stable argsort of -p: ties to the lower id; int64 ids), their weights p / max(sum of the k p, 2^-14) in
    float32."""
    p = softmax(logits) if gating == "softmax" else sigmoid(logits)
    ids = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, axis=-1)
    return ids, (w / np.maximum(w.sum(axis=-1, keepdims=True), MIN_WEIGHT_SUM)).astype(np.float32)


def swiglu(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """down (silu(gate x) * up x) in float32 matrices (``tests/moe/ref.py:21-24``): x (T, H), gate / up (F, H),
    down (H, F)."""
    v = f32(x)
    return (silu(v @ f32(gate).T) * (v @ f32(up).T)) @ f32(down).T


Expert = Callable[[int], tuple[np.ndarray, np.ndarray, np.ndarray]]


def moe_ffn(x: np.ndarray, ids: np.ndarray, weights: np.ndarray, expert: Expert,
            ffn: Callable[..., np.ndarray] = swiglu) -> np.ndarray:
    """The routed experts' sum (``tests/moe/ref.py:43-52``): for each expert e in ascending id order (``np.unique``),
    its (token, slot) pairs in row-major order (``np.nonzero``), y[t] += w[t, i] * ffn_e(x[t]) in float32."""
    v = f32(x)
    y = np.zeros_like(v)
    w = f32(weights)
    for e in np.unique(ids):
        t, i = np.nonzero(ids == e)
        y[t] += w[t, i][:, None] * ffn(v[t], *expert(int(e)))
    return y


def shared_expert(x: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray,
                  gate_inp: np.ndarray | None) -> np.ndarray:
    """The shared expert (``tests/moe/ref.py:55-60``): swiglu(x), times sigmoid(x . gate_inp) when gated (qwen35moe's
    ``ffn_gate_inp_shexp``), else times 1."""
    y = swiglu(x, gate, up, down)
    return y if gate_inp is None else sigmoid(f32(x) @ f32(gate_inp).reshape(-1, 1)) * y
