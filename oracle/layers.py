"""The synthetic MoE layers of the benchmark configurations (seeded), and the oracle's forward pass over them.

A layer holds what a GGUF file holds for one MoE block: the router ``ffn_gate_inp`` (E, H) fp32 and the 3-D expert
tensors as raw blocks, an expert's matrix contiguous (``tests/moe/ref.py:27-40``): ``ffn_gate_exps`` / ``ffn_up_exps``
(E F rows of H values) and ``ffn_down_exps`` (E H rows of F values); optionally a shared expert.

Config 5's skewed routing comes from a constant input feature: x[:, 0] = 1 and router column 0 = a per-expert bias
(Zipf s = 1.2 over 26 experts, -1e4 for 6 that receive no token), so the layer's own arithmetic is unchanged.

Test infrastructure only (see ``oracle/__init__.py``)."""

from dataclasses import dataclass, field

import numpy as np

from . import gguf_ref, host_ref, moe_ref
from .tensors import from_bf16_bits, random_blocks, to_bf16


@dataclass(frozen=True)
class Spec:
    name: str
    H: int
    E: int
    k: int
    F: int
    gate_type: str  # gate / up format
    down_type: str
    scale: float  # fp16 scale std of the expert blocks
    router: str = "normal"  # "normal" N(0, 0.02), "uniform" U(-0.035, 0.035), "zipf" (config 5)
    x_dtype: str = "bf16"  # activations: "bf16" (values of bf16) or "f32"
    shared_F: int = 0  # one shared FFN of this width (0: none)
    shared_type: str = ""  # the shared gate / up format
    shared_gated: bool = False
    tokens: tuple[int, ...] = (16,)
    dmin_scale: float = 0.0  # Q4_K / Q5_K: the fp16 dmin std
    shared_down_type: str = ""  # the shared down's format, when not shared_type's
    shared_scale: float = 0.0  # the shared expert's fp16 scale std (0: scale)

    @property
    def sdown_type(self) -> str:
        return self.shared_down_type or self.shared_type


CONFIGS = {
    "cpu": Spec("cpu", H=1024, E=8, k=2, F=512, gate_type="Q8_0", down_type="Q8_0", scale=0.01, x_dtype="f32",
                tokens=(16,)),
    "decode": Spec("decode", H=2048, E=128, k=8, F=768, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                   tokens=(1, 4, 16, 64)),
    "prefill": Spec("prefill", H=2048, E=128, k=8, F=768, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                    router="uniform", tokens=(4096,)),
    # (the routed down has K = 1408, not a multiple of Q4_K's 256: Q8_0, a 32-block type the reference reads)
    "deepseek": Spec("deepseek", H=2048, E=64, k=6, F=1408, gate_type="Q4_K", down_type="Q8_0", scale=2e-4,
                     dmin_scale=1.5e-3, shared_F=2816, shared_type="Q4_K", tokens=(512,)),
    "skewed": Spec("skewed", H=2880, E=32, k=4, F=2880, gate_type="Q8_0", down_type="Q8_0", scale=0.01,
                   router="zipf", tokens=(2048,)),
    # test-only mixes of the block types at decode sizes (every product on the decode GEMV)
    "mix_q8k": Spec("mix_q8k", H=1024, E=32, k=4, F=512, gate_type="Q8_0", down_type="Q4_K", scale=0.01,
                    dmin_scale=1.5e-3, x_dtype="f32", shared_F=512, shared_type="Q4_K", shared_gated=True,
                    tokens=(16,)),
    "mix_k8": Spec("mix_k8", H=1536, E=16, k=2, F=768, gate_type="Q4_K", down_type="Q8_0", scale=2e-4,
                   dmin_scale=1.5e-3, shared_F=256, shared_type="Q8_0", tokens=(24,)),
    # test-only prefill-sized mix: fp32 x, Q8_0 gate / up, Q4_0 down, a gated Q8_0 shared expert (every product on
    # the prefill tiles)
    "mix_pf": Spec("mix_pf", H=1024, E=16, k=2, F=512, gate_type="Q8_0", down_type="Q4_0", scale=0.01,
                   x_dtype="f32", shared_F=512, shared_type="Q8_0", shared_gated=True, tokens=(256,)),
    # test-only prefill-sized Q4_0 layer with a Q4_0 shared expert twice as wide as the routed ones: on the prefill
    # tiles the shared gate / up joins the routed gate / up launch and the shared down, in two parts of its K, the
    # routed down launch
    "shared_pf": Spec("shared_pf", H=1024, E=16, k=2, F=512, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                      shared_F=1024, shared_type="Q4_0", tokens=(256,)),
    # test-only: Q4_0 with about 128 pairs per expert (T = 512), so the prefill tiles' 8-row-block form runs
    "q4_rows": Spec("q4_rows", H=1024, E=8, k=2, F=512, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                    router="uniform", tokens=(512,)),
    # the same with Q4_K gate / up and down (the prefill tiles' super-block staging in both launches)
    "k4_rows": Spec("k4_rows", H=1024, E=8, k=2, F=512, gate_type="Q4_K", down_type="Q4_K", scale=2e-4,
                    dmin_scale=1.5e-3, router="uniform", tokens=(512,)),
    # test-only: the other block formats of real GGUF files, on the MFMA decode tiles -- K-quants (Q5_K gate / up,
    # Q6_K down, a Q4_K / Q3_K shared expert: 16-value sub-block scales) with bf16 x, and IQ4_XS / IQ4_NL with a
    # Q4_1 shared expert and fp32 x
    "kquants": Spec("kquants", H=1024, E=16, k=2, F=512, gate_type="Q5_K", down_type="Q6_K", scale=1e-4,
                    dmin_scale=1e-3, shared_F=512, shared_type="Q4_K", shared_down_type="Q3_K", tokens=(32,)),
    # test-only: a mixed quantisation as GGUF files store it (Q4_K gate / up, Q6_K down; the shared expert likewise) at
    # decode size: gate / up on the GEMV, the downs on the MFMA decode tiles
    "kmix": Spec("kmix", H=1024, E=32, k=4, F=512, gate_type="Q4_K", down_type="Q6_K", scale=2e-4, dmin_scale=1.5e-3,
                 shared_F=512, shared_type="Q4_K", shared_down_type="Q6_K", shared_gated=True, tokens=(16,)),
    # test-only: Q5_K on the decode GEMV, with a Q6_K routed down (Q5_K_M files) or a Q5_K one
    "q5km": Spec("q5km", H=1024, E=32, k=4, F=512, gate_type="Q5_K", down_type="Q6_K", scale=1e-4, dmin_scale=1e-3,
                 shared_F=512, shared_type="Q5_K", tokens=(16,)),
    "q5k": Spec("q5k", H=1536, E=16, k=2, F=768, gate_type="Q5_K", down_type="Q5_K", scale=1e-4, dmin_scale=1e-3,
                x_dtype="f32", tokens=(24,)),
    # test-only: Q6_K throughout on the decode GEMV; a Q4_K gate / up with a Q3_K down
    "q6k": Spec("q6k", H=1024, E=16, k=2, F=512, gate_type="Q6_K", down_type="Q6_K", scale=5e-5, x_dtype="f32",
                shared_F=256, shared_type="Q6_K", tokens=(24,)),
    "mixtile": Spec("mixtile", H=1024, E=32, k=4, F=512, gate_type="Q4_K", down_type="Q3_K", scale=2e-4,
                    dmin_scale=1.5e-3, tokens=(16,)),
    "iq4": Spec("iq4", H=768, E=16, k=4, F=512, gate_type="IQ4_XS", down_type="IQ4_NL", scale=5e-5, x_dtype="f32",
                shared_F=256, shared_type="Q4_1", shared_scale=4e-3, shared_gated=True, tokens=(16, 24)),
    # test-only: Q3_K throughout on the decode GEMV (16-value sub-block scales, 3-bit codes), fp32 x
    "q3k": Spec("q3k", H=1024, E=16, k=2, F=512, gate_type="Q3_K", down_type="Q3_K", scale=1e-4, x_dtype="f32",
                shared_F=256, shared_type="Q3_K", tokens=(16,)),
    # test-only: Q4_1 throughout (d q + m blocks: the min term) with an IQ4_XS / IQ4_NL shared expert
    "q41": Spec("q41", H=1024, E=16, k=2, F=512, gate_type="Q4_1", down_type="Q4_1", scale=4e-3, shared_F=256,
                shared_type="IQ4_XS", shared_down_type="IQ4_NL", shared_scale=5e-5, tokens=(16,)),
    # test-only: an expert width of 256 (the down's K below the prefill tiles' 320), so that passes past the GEMV's
    # sizes take the MFMA decode tiles
    "dtiles": Spec("dtiles", H=1024, E=16, k=2, F=256, gate_type="Q4_K", down_type="Q6_K", scale=2e-4,
                   dmin_scale=1.5e-3, tokens=(96,)),
    # test-only: top 16 of 160 experts, so that 33 to 40 decode tokens (more pairs than a GEMV workgroup routes) take
    # the routing launch of their own
    "widek": Spec("widek", H=512, E=160, k=16, F=256, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                  tokens=(16, 40)),
    # test-only: top 20 of 64 experts, past the 16 a lane group takes, so that the gate / up launch's routing takes
    # the top k a wave per token
    "topk20": Spec("topk20", H=512, E=64, k=20, F=256, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                   tokens=(12,)),
    # test-only: 320 experts (eight logits a lane in the gate / up launch's top k)
    "wide_e": Spec("wide_e", H=256, E=320, k=4, F=256, gate_type="Q4_0", down_type="Q4_0", scale=0.02,
                   tokens=(16,)),
    # the Qwen3-30B-A3B shape as Q4_K_M files quantise it (Q4_K gate / up, Q6_K down) at a 4096-token prefill: the
    # down on the prefill tiles through the prefill layout
    "q4km": Spec("q4km", H=2048, E=128, k=8, F=768, gate_type="Q4_K", down_type="Q6_K", scale=2e-4, dmin_scale=1.5e-3,
                 router="uniform", tokens=(4096,)),
}

ZIPF_S, ZIPF_ACTIVE, ZIPF_BETA = 1.2, 26, 0.7


@dataclass
class Layer:
    spec: Spec
    router: np.ndarray  # (E, H) fp32
    gate: np.ndarray  # (E F, row bytes of H) uint8
    up: np.ndarray
    down: np.ndarray  # (E H, row bytes of F) uint8
    shared: tuple[np.ndarray, np.ndarray, np.ndarray] | None = None
    shared_inp: np.ndarray | None = None  # (H,) fp32 gate of a gated shared expert
    meta: dict = field(default_factory=dict)


def _blocks(qtype: str, rows: int, cols: int, rng: np.random.Generator, spec: Spec, scale: float = 0.0) -> np.ndarray:
    raw = random_blocks(qtype, rows, cols, rng, scale=scale or spec.scale, abs_scales=True)
    if qtype in ("Q4_K", "Q5_K"):  # (dmin: its own, larger scale, so the weights are about centred)
        n, nb = cols // 256, gguf_ref.BLOCKS[qtype][1]
        dmin = (np.abs(rng.standard_normal((rows, n))) * spec.dmin_scale).astype(np.float16)
        raw.reshape(rows, n, nb)[..., 2:4] = dmin.view(np.uint8).reshape(rows, n, 2)
    return raw


def make_layer(spec: Spec, seed: int = 0) -> Layer:
    """The layer of ``spec`` from ``seed``: router N(0, 0.02) (``uniform``: U(-0.035, 0.035); ``zipf``: plus the bias
    column), expert blocks of ``random_blocks`` with |N(0, scale)| fp16 scales."""
    rng = np.random.default_rng(seed)
    H, E, F = spec.H, spec.E, spec.F
    if spec.router == "uniform":
        router = rng.uniform(-0.035, 0.035, (E, H)).astype(np.float32)
    else:
        router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    meta = {}
    if spec.router == "zipf":
        bias = np.full(E, -1e4, np.float64)
        perm = np.random.default_rng(seed + 1).permutation(E)
        bias[perm[:ZIPF_ACTIVE]] = ZIPF_BETA * -ZIPF_S * np.log(np.arange(1, ZIPF_ACTIVE + 1))
        router[:, 0] = bias.astype(np.float32)
        meta["cold"] = np.sort(perm[ZIPF_ACTIVE:])
    gate = _blocks(spec.gate_type, E * F, H, rng, spec)
    up = _blocks(spec.gate_type, E * F, H, rng, spec)
    down = _blocks(spec.down_type, E * H, F, rng, spec)
    shared = None
    if spec.shared_F:
        Fs = spec.shared_F
        sc = spec.shared_scale
        shared = (_blocks(spec.shared_type, Fs, H, rng, spec, sc), _blocks(spec.shared_type, Fs, H, rng, spec, sc),
                  _blocks(spec.sdown_type, H, Fs, rng, spec, sc))
    shared_inp = (rng.standard_normal(H) * 0.02).astype(np.float32) if spec.shared_gated else None
    return Layer(spec, router, gate, up, down, shared, shared_inp, meta)


def make_x(spec: Spec, T: int, seed: int = 0) -> np.ndarray:
    """(T, H) fp32 activations N(0, 1) (bf16 values for ``x_dtype`` "bf16"); ``zipf``: feature 0 the constant 1."""
    x = np.random.default_rng(10_000 + seed).standard_normal((T, spec.H)).astype(np.float32)
    if spec.router == "zipf":
        x[:, 0] = 1.0
    return to_bf16(x) if spec.x_dtype == "bf16" else x


def expert(layer: Layer):
    """``tests/moe/ref.py:27-40``'s ``experts``: expert e's (gate (F, H), up (F, H), down (H, F)) dequantized to fp32
    on demand from its rows of the 3-D tensors."""
    s = layer.spec

    def get(e: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        g = gguf_ref.dequantize(s.gate_type, layer.gate[e * s.F:(e + 1) * s.F], s.H)
        u = gguf_ref.dequantize(s.gate_type, layer.up[e * s.F:(e + 1) * s.F], s.H)
        d = gguf_ref.dequantize(s.down_type, layer.down[e * s.H:(e + 1) * s.H], s.F)
        return g, u, d

    return get


def logits(layer: Layer, x: np.ndarray) -> np.ndarray:
    """Router logits as the reference's decode test computes them (``tests/qwen35/test_decode.py:1073``): x W^T in
    float64, rounded to fp32."""
    return (np.asarray(x, np.float64) @ layer.router.astype(np.float64).T).astype(np.float32)


def shared_out(layer: Layer, x: np.ndarray) -> np.ndarray:
    """The shared expert's output (``tests/moe/ref.py:55-60``), zeros without one."""
    s = layer.spec
    if layer.shared is None:
        return np.zeros((x.shape[0], s.H), np.float32)
    g, u, d = layer.shared
    return moe_ref.shared_expert(x, gguf_ref.dequantize(s.shared_type, g, s.H),
                                 gguf_ref.dequantize(s.shared_type, u, s.H),
                                 gguf_ref.dequantize(s.sdown_type, d, s.shared_F), layer.shared_inp)


def forward(layer: Layer, x: np.ndarray, ids: np.ndarray | None = None, w: np.ndarray | None = None,
            gating: str = "softmax") -> dict:
    """The oracle's layer: logits (``logits``), the routing of ``moe_ref.moe_route`` (or the given ids / w), the routed
    sum ``moe_ref.moe_ffn`` plus the shared expert. Returns logits, ids, w, y (T, H) fp32."""
    lg = logits(layer, x)
    if ids is None:
        ids, w = moe_ref.moe_route(lg, layer.spec.k, gating)
    y = moe_ref.moe_ffn(x, ids, w, expert(layer)) + shared_out(layer, x)
    return {"logits": lg, "ids": ids, "w": w, "y": y}


def forward_f64(layer: Layer, x: np.ndarray, ids: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The same layer for a given routing in float64 throughout (a second reference for the tolerance tests)."""
    s = layer.spec
    xv = np.asarray(x, np.float64)
    y = np.zeros_like(xv)
    get = expert(layer)

    def ffn(xs: np.ndarray, g: np.ndarray, u: np.ndarray, d: np.ndarray) -> np.ndarray:
        a = xs @ g.astype(np.float64).T
        return ((a / (1.0 + np.exp(-a))) * (xs @ u.astype(np.float64).T)) @ d.astype(np.float64).T

    for e in np.unique(ids):
        t, i = np.nonzero(ids == e)
        y[t] += np.asarray(w, np.float64)[t, i][:, None] * ffn(xv[t], *get(int(e)))
    if layer.shared is not None:
        g, u, d = layer.shared
        ys = ffn(xv, gguf_ref.dequantize(s.shared_type, g, s.H), gguf_ref.dequantize(s.shared_type, u, s.H),
                 gguf_ref.dequantize(s.sdown_type, d, s.shared_F))
        if layer.shared_inp is not None:
            ys = ys / (1.0 + np.exp(-(xv @ layer.shared_inp.astype(np.float64))))[:, None]
        y += ys
    return y


def route_host(layer: Layer, lg: np.ndarray, gating: str = "softmax") -> tuple[np.ndarray, np.ndarray]:
    """The C++ host routing (``host_ref.moe_route``) of plain (T, E) logits."""
    T, E = lg.shape
    return host_ref.moe_route(lg.reshape(-1), T, E, E, 0, E, layer.spec.k, sigmoid=gating == "sigmoid")


def tie_collapsed(lg: np.ndarray, k: int, gating: str = "softmax") -> np.ndarray:
    """Tokens whose probability ranking can differ from their logit ranking: two of their k + 1 largest logits are
    distinct but have equal fp32 probabilities, softmax or (gating "sigmoid") sigmoid (the oracle ranks by p, the host
    step by logit)."""
    from .np_ops import sigmoid, softmax

    p = softmax(lg) if gating == "softmax" else sigmoid(lg)
    order = np.argsort(-host_ref.ordered_keys(lg).astype(np.int64), axis=1, kind="stable")[:, :k + 1]
    lt = np.take_along_axis(lg, order, 1)
    pt = np.take_along_axis(p, order, 1)
    return ((lt[:, :-1] != lt[:, 1:]) & (pt[:, :-1] == pt[:, 1:])).any(axis=1)


__all__ = ["CONFIGS", "Layer", "Spec", "expert", "forward", "forward_f64", "from_bf16_bits", "logits", "make_layer",
           "make_x", "route_host", "shared_out", "tie_collapsed"]
