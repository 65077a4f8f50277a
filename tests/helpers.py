"""Shared test helpers: an oracle layer uploaded into a GPU ``MoELayer``, comparators."""

import numpy as np

from artlite_amd.moe.layer import MoELayer
from oracle import layers
from oracle.tensors import bf16_bits


def layer_args(s: layers.Spec, max_tokens: int, gating: str = "softmax") -> dict:
    """``MoELayer``'s keyword arguments for an oracle configuration."""
    return dict(hidden=s.H, n_experts=s.E, top_k=s.k, expert_ffn=s.F, gate_type=s.gate_type, down_type=s.down_type,
                max_tokens=max_tokens, shared_ffn=s.shared_F, shared_type=s.shared_type, shared_gated=s.shared_gated,
                shared_down_type=s.shared_down_type, gating=gating)


def gpu_layer(layer: layers.Layer, max_tokens: int, gating: str = "softmax") -> MoELayer:
    g = MoELayer(**layer_args(layer.spec, max_tokens, gating))
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


def near_tie(lg_ref: np.ndarray, k: int, gating: str = "softmax") -> np.ndarray:
    """Tokens whose k-th / (k + 1)-th choice the oracle may order differently from the logits: a gap within 1e-5 of
    the row's scale among the k + 1 largest logits, or distinct logits with equal fp32 probabilities."""
    srt = np.sort(lg_ref, axis=1)[:, ::-1]
    gap = srt[:, :k] - srt[:, 1:k + 1]
    near = (gap < 1e-5 * np.abs(srt[:, :k + 1]).max(1, keepdims=True)).any(1)
    return near | layers.tie_collapsed(lg_ref, k, gating)


def check_against_oracle(g: MoELayer, layer: layers.Layer, x: np.ndarray, y: np.ndarray, *,
                         gating: str = "softmax") -> dict:
    """The GPU layer's last run of x against the oracle: logits within one ulp (float64 accumulation on both sides);
    ids bit-exact against the C++ host routing of the GPU's logits, weights within one ulp of it; ids equal to the
    layer oracle's own routing except at near ties; counts, offsets, order and slots bit-exact against the stable
    counting sort; y within 1e-3 relative L2 of the fp32 oracle for the GPU's routing. Returns the taps read."""
    from oracle import host_ref, moe_ref

    spec = layer.spec
    lg, ids, w = g.tap("logits"), g.tap("ids"), g.tap("weights")
    lg_ref = layers.logits(layer, x)
    d = ulp_diff(lg, lg_ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.999, (d.max(), (d == 0).mean())
    hids, hw = layers.route_host(layer, lg, gating)
    assert np.array_equal(ids, hids)
    assert ulp_diff(w, hw).max() <= 1
    rids, _ = moe_ref.moe_route(lg_ref, spec.k, gating)
    near = near_tie(lg_ref, spec.k, gating)
    assert near.mean() < 0.01 and np.array_equal(ids[~near], rids[~near])
    dref = host_ref.dispatch(ids, spec.E)
    taps = {"logits": lg, "ids": ids, "weights": w}
    for tap in ("counts", "offsets", "order", "slot"):
        taps[tap] = g.tap(tap)
        assert np.array_equal(taps[tap], dref[tap]), tap
    want = moe_ref.moe_ffn(x, ids, w, layers.expert(layer)) + layers.shared_out(layer, x)
    err = rel_l2(y, want)
    assert err < 1e-3, err
    taps["rel_l2"] = err
    return taps


def check_pairs_f64(g: MoELayer, layer: layers.Layer, x: np.ndarray, offsets: np.ndarray, order: np.ndarray,
                    experts: list[int], tol: float) -> None:
    """For each listed expert, its sorted pairs' h = silu(x G^T) (x U^T) (tap "h") and expert outputs (tap
    "y_pairs") against float64 math on the oracle's dequantized weights, within ``tol`` relative L2."""
    spec = layer.spec
    get = layers.expert(layer)
    h, yp = g.tap("h"), g.tap("y_pairs")
    x64 = np.asarray(x, np.float64)
    for e in experts:
        s0, s1 = int(offsets[e]), int(offsets[e + 1])
        if s0 == s1:
            continue
        gw, uw, dw = (m.astype(np.float64) for m in get(int(e)))
        xt = x64[order[s0:s1] // spec.k]
        a = xt @ gw.T
        h64 = a / (1 + np.exp(-a)) * (xt @ uw.T)
        assert rel_l2(h[s0:s1], h64) < tol, (e, s1 - s0, rel_l2(h[s0:s1], h64))
        assert rel_l2(yp[s0:s1], h64 @ dw.T) < tol, (e, s1 - s0, rel_l2(yp[s0:s1], h64 @ dw.T))
