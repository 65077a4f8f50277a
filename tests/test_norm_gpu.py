"""The steps either side of the block: RMSNorm of x before the router (``ffn_norm``; the reference's rms_norm,
tests/np_ops.py:27-32) and the residual add after the combine, on the GPU against the oracle."""

import numpy as np
import pytest

from oracle import layers, moe_ref, np_ops

from .helpers import gpu_input, layer_args, rel_l2, ulp_diff

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(("name", "T"), [("decode", 16), ("prefill", 256), ("mix_pf", 256), ("deepseek", 64)])
def test_norm_and_residual(name: str, T: int) -> None:
    from artlite_amd.moe.layer import MoELayer

    spec = layers.CONFIGS[name]
    layer = layers.make_layer(spec, 7)
    x = layers.make_x(spec, T, 7) * np.float32(3.0)  # (a row RMS away from 1)
    w = np.random.default_rng(7).normal(1.0, 0.1, spec.H).astype(np.float32)
    eps = 1e-6
    s = spec
    with MoELayer(**layer_args(s, T), norm_eps=eps, residual=True) as g:
        for n, t in (("ffn_gate_inp", layer.router), ("ffn_gate_exps", layer.gate), ("ffn_up_exps", layer.up),
                     ("ffn_down_exps", layer.down), ("ffn_norm", w)):
            g.upload(n, t)
        if layer.shared is not None:
            for n, t in zip(("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"), layer.shared):
                g.upload(n, t)
        if layer.shared_inp is not None:
            g.upload("ffn_gate_inp_shexp", layer.shared_inp)
        xi = gpu_input(spec, x)
        y = g(xi)
        xn, ids, wts = g.tap("x_norm"), g.tap("ids"), g.tap("weights")
        assert "rmsnorm" in g.kernel_names()
    xv = layers.from_bf16_bits(xi) if xi.dtype == np.uint16 else xi
    xn_ref = np_ops.rms_norm(xv, w, eps)
    d = ulp_diff(xn, xn_ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.999, (d.max(), (d == 0).mean())
    # the block on the normalised x (the GPU's routing), plus the residual
    want = moe_ref.moe_ffn(xn, ids, wts, layers.expert(layer)) + layers.shared_out(layer, xn) + xv
    assert rel_l2(y, want) < 1e-3, rel_l2(y, want)


def test_norm_errors() -> None:
    from artlite_amd import Error
    from artlite_amd.moe.layer import MoELayer

    spec = layers.CONFIGS["cpu"]
    with pytest.raises(Error):
        MoELayer(hidden=spec.H, n_experts=spec.E, top_k=spec.k, expert_ffn=spec.F, gate_type=spec.gate_type,
                 down_type=spec.down_type, max_tokens=4, norm_eps=-1.0)
    layer = layers.make_layer(spec, 0)
    with MoELayer(hidden=spec.H, n_experts=spec.E, top_k=spec.k, expert_ffn=spec.F, gate_type=spec.gate_type,
                  down_type=spec.down_type, max_tokens=4, norm_eps=1e-6) as g:
        for n, t in (("ffn_gate_inp", layer.router), ("ffn_gate_exps", layer.gate), ("ffn_up_exps", layer.up),
                     ("ffn_down_exps", layer.down)):
            g.upload(n, t)
        with pytest.raises(Error, match="ffn_norm"):
            g(np.zeros((2, spec.H), np.float32))
