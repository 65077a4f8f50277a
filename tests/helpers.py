"""Shared test helpers: an oracle layer uploaded into a GPU ``MoELayer``, comparators."""

import numpy as np

from artlite_amd.moe.layer import MoELayer
from oracle import layers
from oracle.tensors import bf16_bits


def layer_args(s: layers.Spec, max_tokens: int) -> dict:
    """``MoELayer``'s keyword arguments for an oracle configuration."""
    return dict(hidden=s.H, n_experts=s.E, top_k=s.k, expert_ffn=s.F, gate_type=s.gate_type, down_type=s.down_type,
                max_tokens=max_tokens, shared_ffn=s.shared_F, shared_type=s.shared_type, shared_gated=s.shared_gated,
                shared_down_type=s.shared_down_type)


def gpu_layer(layer: layers.Layer, max_tokens: int) -> MoELayer:
    g = MoELayer(**layer_args(layer.spec, max_tokens))
    g.upload("ffn_gate_inp", layer.router)
    g.upload("ffn_gate_exps", layer.gate)
    g.upload("ffn_up_exps", layer.up)
    g.upload("ffn_down_exps", layer.down)
    if layer.shared is not None:
        g.upload("ffn_gate_shexp", layer.shared[0])
        g.upload("ffn_up_shexp", layer.shared[1])
        g.upload("ffn_down_shexp", layer.shared[2])
    if layer.shared_inp is not None:
        g.upload("ffn_gate_inp_shexp", layer.shared_inp)
    return g


def gpu_input(spec: layers.Spec, x: np.ndarray) -> np.ndarray:
    """x as the layer takes it: bf16 bit patterns for bf16 configurations (x holds bf16 values), else fp32."""
    return bf16_bits(x) if spec.x_dtype == "bf16" else np.ascontiguousarray(x, np.float32)


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    """|got - want| / |want| (Frobenius, float64)."""
    g, w = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(g - w) / np.linalg.norm(w))


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in units of the last place of float32 (ordered-integer distance)."""
    def key(v: np.ndarray) -> np.ndarray:
        u = np.asarray(v, np.float32).view(np.int32).astype(np.int64)
        return np.where(u < 0, -(u & 0x7FFFFFFF), u)

    return np.abs(key(a) - key(b))
