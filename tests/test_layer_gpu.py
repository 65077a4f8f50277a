"""The GPU MoE layer against the oracle, stage by stage through its taps, on every benchmark configuration:

- router logits: float64 accumulation on both sides, so bit-exact fp32 logits (a rounding-boundary tie may differ by
  one ulp);
- routing: ids bit-exact against the C++ host routing's restatement applied to the GPU's logits, weights within one
  fp32 ulp; ids equal to the layer oracle's (by probability, on its own logits) except where a near-tie leaves the
  order to rounding;
- dispatch: counts, offsets, sorted order and slots bit-exact against the stable counting sort of the GPU's ids;
- experts: h = silu(x G^T) (x U^T) of each sorted pair and each pair's expert output against float64 math;
- output: within 1e-3 relative L2 of the fp32 oracle (``moe_ffn`` + ``shared_expert``) and of float64 math for the
  same routing; bitwise identical on a second run (deterministic kernels, no float atomics).
Config sizes are reduced here; test_layer_full_gpu.py runs configs 3, 4 and 5 at their stated sizes."""

import numpy as np
import pytest

from artlite_amd.moe.layer import MoELayer
from oracle import gguf_ref, host_ref, layers, moe_ref

from .helpers import check_against_oracle, gpu_input, gpu_layer, near_tie, rel_l2, ulp_diff

pytestmark = pytest.mark.gpu

CASES = [("cpu", 16), ("decode", 1), ("decode", 4), ("decode", 16), ("decode", 64), ("prefill", 256),
         ("deepseek", 64), ("skewed", 192), ("mix_q8k", 16), ("mix_k8", 24), ("mix_pf", 256), ("shared_pf", 256),
         ("kquants", 32),
         ("kquants", 160), ("iq4", 24), ("iq4", 96), ("kmix", 16), ("kmix", 64),
         ("q5km", 16), ("q5k", 24), ("q6k", 24), ("mixtile", 16), ("iq4", 16), ("q41", 16), ("q3k", 16),
         # prefill-sized passes of the formats the prefill tiles read through the prefill layout
         ("kmix", 160), ("q5km", 160), ("q5k", 160), ("q6k", 192), ("mixtile", 160), ("q3k", 160), ("q41", 160),
         # past the GEMV's sizes with a down the prefill tiles do not take (K = 256): the MFMA decode tiles
         ("dtiles", 96),
         # the decode routing in a launch of its own (more pairs than a GEMV workgroup routes), and in the GEMV's
         ("widek", 40), ("widek", 16),
         # the routing in the gate / up launch with a wave per token (top 20: more than a lane group takes)
         ("topk20", 12), ("wide_e", 16),
         # 320 and 160 experts past the GEMV's sizes (the MFMA decode tiles): the router's K in parts that the top-k
         # launch adds, eight and four logits a lane
         ("wide_e", 384), ("widek", 256)]
# (passes on the MFMA decode tiles)
DTILE_CASES = {("dtiles", 96), ("wide_e", 384), ("widek", 256)}

# Decode-sized passes (at most 4 pairs per expert on average, K a multiple of 256) take the GEMV over XQ activations:
# int8 hi / lo planes per 32 values, |x - xq| <= max|x| / 65024 per group, so h (itself held in XQ) and the pair
# outputs carry a few 1e-5 of relative error; the MFMA decode tiles' bf16 hi / lo planes, about 2^-17. Larger passes
# take the prefill tiles' fp16 products: weights d (q - 8) and h rounded once to fp16 (2^-11 relative at most), a few
# 1e-4 of relative error in h and the pair outputs.
GEMV_CASES = {("cpu", 16), ("decode", 1), ("decode", 4), ("decode", 16), ("decode", 64), ("mix_q8k", 16), ("mix_k8", 24),
              ("kmix", 16), ("q5km", 16), ("q5k", 24), ("kquants", 32), ("q6k", 24), ("mixtile", 16), ("iq4", 16),
              ("q41", 16), ("q3k", 16), ("widek", 40), ("widek", 16), ("topk20", 12), ("wide_e", 16)}


def check_layer(name: str, T: int, seed: int = 0) -> None:
    spec = layers.CONFIGS[name]
    layer = layers.make_layer(spec, seed)
    x = layers.make_x(spec, T, seed)
    with gpu_layer(layer, max_tokens=T) as g:
        y = g(gpu_input(spec, x))
        gemv = any(n.startswith("router_quant") for n in g.kernel_names())
        prefill = "prefill_x" in g.kernel_names()
        assert gemv == ((name, T) in GEMV_CASES), (name, T, g.kernel_names())
        if name in ("shared_pf", "mix_pf"):  # (the shared gate / up in the routed launch; the down too when alike)
            assert "shared_gate_up" not in g.kernel_names(), g.kernel_names()
            assert ("shared_down" in g.kernel_names()) == (name == "mix_pf"), g.kernel_names()
        # (every block format has prefill tiles: every pass past the GEMV's sizes takes them where they take its shapes)
        assert prefill == (not gemv and (name, T) not in DTILE_CASES), (name, T, g.kernel_names())
        tol = 1e-4 if gemv else 1e-3 if prefill else 1e-5
        lg = g.tap("logits")
        ids, w = g.tap("ids"), g.tap("weights")
        # logits
        lg_ref = layers.logits(layer, x)
        d = ulp_diff(lg, lg_ref)
        assert d.max() <= 1 and (d == 0).mean() > 0.999, (name, T, d.max(), (d == 0).mean())
        # routing of the GPU's logits: the host step's semantics, bit for bit
        hids, hw = layers.route_host(layer, lg)
        assert np.array_equal(ids, hids), name
        assert ulp_diff(w, hw).max() <= 1
        # the layer oracle's own routing: equal but where a near-tie leaves it to rounding
        rids, rw = moe_ref.moe_route(lg_ref, spec.k)
        srt = np.sort(lg_ref, axis=1)[:, ::-1]
        gap = srt[:, :spec.k] - srt[:, 1:spec.k + 1]
        near = (gap < 1e-5 * np.abs(srt[:, :spec.k]).max(1, keepdims=True)).any(1) | layers.tie_collapsed(lg_ref,
                                                                                                       spec.k)
        assert np.array_equal(ids[~near], rids[~near]), name
        # dispatch
        dref = host_ref.dispatch(ids, spec.E)
        for tap in ("counts", "offsets", "order", "slot"):
            assert np.array_equal(g.tap(tap), dref[tap]), tap
        # experts: per sorted pair, h and the expert output against float64 math
        get = layers.expert(layer)
        order = dref["order"]
        h, yp = g.tap("h"), g.tap("y_pairs")
        x64 = x.astype(np.float64)
        for e in np.unique(ids)[:6]:
            s0, s1 = dref["offsets"][e], dref["offsets"][e + 1]
            gw, uw, dw = (m.astype(np.float64) for m in get(int(e)))
            xt = x64[order[s0:s1] // spec.k]
            a = xt @ gw.T
            h64 = a / (1 + np.exp(-a)) * (xt @ uw.T)
            assert rel_l2(h[s0:s1], h64) < tol, (name, e, rel_l2(h[s0:s1], h64))
            assert rel_l2(yp[s0:s1], h64 @ dw.T) < max(tol, 1e-4), (name, e, rel_l2(yp[s0:s1], h64 @ dw.T))
        # the shared expert's output (before its gate) against float64 math
        if layer.shared is not None:
            sg, su, sd = (gguf_ref.dequantize(q, m, c).astype(np.float64) for q, m, c in
                          zip((spec.shared_type, spec.shared_type, spec.sdown_type), layer.shared,
                              (spec.H, spec.H, spec.shared_F)))
            a = x64 @ sg.T
            ys64 = (a / (1 + np.exp(-a)) * (x64 @ su.T)) @ sd.T
            assert rel_l2(g.tap("y_shared"), ys64) < (1e-3 if prefill else max(tol, 1e-4)), name
        # output: the fp32 oracle and float64 math for the GPU's routing
        want = moe_ref.moe_ffn(x, ids, w, get) + layers.shared_out(layer, x)
        assert rel_l2(y, want) < 1e-3, (name, T, rel_l2(y, want))
        y64 = layers.forward_f64(layer, x, ids, w)
        assert rel_l2(y, y64) < 1e-3, (name, T, rel_l2(y, y64))
        # determinism
        assert np.array_equal(g(gpu_input(spec, x)).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize(("name", "T"), CASES)
def test_layer(name: str, T: int) -> None:
    check_layer(name, T)


def test_layer_token_counts() -> None:
    """One layer object for several token counts in turn (buffers sized for the largest), zero tokens included."""
    spec = layers.CONFIGS["decode"]
    layer = layers.make_layer(spec, 3)
    with gpu_layer(layer, max_tokens=40) as g:
        assert g(np.zeros((0, spec.H), np.uint16)).shape == (0, spec.H)
        for T in (40, 3, 17):
            x = layers.make_x(spec, T, T)
            y = g(gpu_input(spec, x))
            ids, w = g.tap("ids"), g.tap("weights")
            assert rel_l2(y, layers.forward_f64(layer, x, ids, w)) < 1e-3


@pytest.mark.parametrize(("name", "counts", "in_gemv"), [("decode", (16, 1, 64, 7, 40, 16, 64, 7), True),
                                                         ("widek", (40, 16, 33, 40), None)])
def test_decode_routing_repeat(name: str, counts: tuple, in_gemv: bool | None) -> None:
    """The decode routing several times in a row, token counts changing between calls (one to four router token
    groups): the few-token router's logits, then the top k and dispatch in every workgroup of the gate / up GEMV's
    launch (workgroup 0 storing them), or, past the pairs a GEMV workgroup routes (``widek``: top 16 of 160 experts,
    more than 512 pairs at 40 tokens), in a one-workgroup launch of their own. Each call's routing and dispatch equal
    the host restatement's, and a repeated input gives bitwise the same output."""
    spec = layers.CONFIGS[name]
    layer = layers.make_layer(spec, 5)
    outs = {}
    with gpu_layer(layer, max_tokens=max(counts)) as g:
        for T in counts:
            x = layers.make_x(spec, T, T)
            y = g(gpu_input(spec, x))
            names = g.kernel_names()
            assert "router_quant" in names, names
            assert ("route" not in names) == (in_gemv if in_gemv is not None else T * spec.k <= 512), (T, names)
            lg, ids, w = g.tap("logits"), g.tap("ids"), g.tap("weights")
            assert ulp_diff(lg, layers.logits(layer, x)).max() <= 1
            hids, hw = layers.route_host(layer, lg)
            assert np.array_equal(ids, hids) and ulp_diff(w, hw).max() <= 1, T
            dref = host_ref.dispatch(ids, spec.E)
            for tap in ("counts", "offsets", "order", "slot"):
                assert np.array_equal(g.tap(tap), dref[tap]), (T, tap)
            assert rel_l2(y, moe_ref.moe_ffn(x, ids, w, layers.expert(layer))) < 1e-3, T
            if T in outs:
                assert np.array_equal(outs[T].view(np.uint32), y.view(np.uint32)), T
            outs[T] = y


def test_layer_errors() -> None:
    from artlite_amd import Error
    from artlite_amd.moe.layer import MoELayer

    with pytest.raises(Error, match="K of E|of E"):
        MoELayer(hidden=64, n_experts=4, top_k=5, expert_ffn=32, gate_type="Q4_0", down_type="Q4_0", max_tokens=4)
    g = MoELayer(hidden=64, n_experts=4, top_k=2, expert_ffn=32, gate_type="Q4_0", down_type="Q4_0", max_tokens=4)
    with pytest.raises(Error, match="not uploaded"):
        g(np.zeros((2, 64), np.float32))
    with pytest.raises(Error, match="is 10 bytes, not 1024"):
        g.upload("ffn_gate_inp", np.zeros(10, np.uint8))
    with pytest.raises(Error, match="5 tokens of at most 4"):
        g.stage(np.zeros((5, 64), np.float32))
    g.close()


@pytest.mark.parametrize(("name", "T"), [("decode", 16), ("mix_pf", 256), ("dtiles", 96), ("q4_rows", 512)])
def test_layer_sigmoid_gating(name: str, T: int) -> None:
    """Sigmoid gating over the whole layer (the GEMV, the prefill tiles, the MFMA decode tiles) against the oracle's
    ``moe_route(gating="sigmoid")`` and the C++ host routing's sigmoid mode."""
    spec = layers.CONFIGS[name]
    layer = layers.make_layer(spec, 11)
    x = layers.make_x(spec, T, 11)
    with gpu_layer(layer, max_tokens=T, gating="sigmoid") as g:
        y = g(gpu_input(spec, x))
        taps = check_against_oracle(g, layer, x, y, gating="sigmoid")
    lg = layers.logits(layer, x)
    want = layers.forward(layer, x, gating="sigmoid")
    near = near_tie(lg, spec.k, "sigmoid")
    assert np.array_equal(taps["ids"][~near], want["ids"][~near])
    s = 1 / (1 + np.exp(-np.take_along_axis(lg, taps["ids"], 1).astype(np.float64)))
    np.testing.assert_allclose(taps["weights"], s / np.maximum(s.sum(1, keepdims=True), 2.0 ** -14), rtol=3e-7)


def test_prefill_offset_guard() -> None:
    """The prefill tiles address an expert tensor and the rows of A with 32-bit offsets: a layer whose Q8_0 gate tensor
    passes 4 GiB (256 experts of 4096 x 4096) takes the MFMA decode tiles at prefill sizes instead, while the same layer
    with 128 experts (2.1 GiB) takes the prefill tiles. (No weights are uploaded: the path is chosen at creation.)"""
    H = F = 4096
    T = 4096
    x = np.zeros((T, H), np.uint16)
    for E, prefill in ((128, True), (256, False)):
        with MoELayer(hidden=H, n_experts=E, top_k=8, expert_ffn=F, gate_type="Q8_0", down_type="Q8_0",
                      max_tokens=T) as g:
            g.stage(x)
            assert ("prefill_x" in g.kernel_names()) == prefill, (E, g.kernel_names())
