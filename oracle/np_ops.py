"""float32 numpy ops of the reference's CPU oracles (restating ``tests/np_ops.py``; tokens first, features last).

Test infrastructure only (see ``oracle/__init__.py``)."""

import numpy as np


def f32(x: object) -> np.ndarray:
    """``tests/np_ops.py:6-7``: an array as float32."""
    return np.asarray(x, np.float32)


def silu(x: np.ndarray) -> np.ndarray:
    """x / (1 + e^-x) in float32 (``tests/np_ops.py:10-12``)."""
    v = f32(x)
    with np.errstate(over="ignore"):  # (e^-x overflows to inf for x < -88: x / inf = -0, the limit)
        return v / (np.float32(1.0) + np.exp(-v))


def sigmoid(x: np.ndarray) -> np.ndarray:
    """1 / (1 + e^-x) in float32 (``tests/np_ops.py:15-17``)."""
    v = f32(x)
    with np.errstate(over="ignore"):
        return np.float32(1.0) / (np.float32(1.0) + np.exp(-v))


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) (the mean in float64) times w (``tests/np_ops.py:27-32``)."""
    v = f32(x)
    ms = (v.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    y = (v / np.sqrt(ms + eps)).astype(np.float32)
    return y if w is None else y * f32(w)


def softmax(x: np.ndarray) -> np.ndarray:
    """Softmax over the last axis as ggml_soft_max (``tests/np_ops.py:35-39``): e = exp(x - max) in float32, the
    sum of e in float64, the quotient rounded to float32."""
    v = f32(x)
    e = np.exp(v - v.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float64)).astype(np.float32)
