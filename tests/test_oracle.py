"""Pins the CPU oracle before anything is checked against it: against the reference's own compiled dequantizer and
its outputs committed under tests/golden, the known answers of the reference's tests (tests/moe/test_route.py,
tests/moe/test_plan.py), closed forms, brute force on tiny inputs, and properties chosen so that a plausible slip (a
dropped offset, a swapped nibble half, a sequential instead of pairwise sum, an unstable sort) fails."""

import dataclasses
import itertools
from pathlib import Path

import numpy as np
import pytest

from oracle import gguf_ref, host_ref, layers, moe_ref, np_ops, ref_lib, tensors

from . import known_answers

GOLDEN = Path(__file__).resolve().parent / "golden" / "dequant_golden.npz"
QTYPES = ("Q4_0", "Q4_1", "Q8_0", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ4_NL", "IQ4_XS")


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


# ---- dequantization


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_golden(qtype: str) -> None:
    """The numpy dequant equals the reference C++ outputs committed in tests/golden (random and edge blocks)."""
    z = np.load(GOLDEN)
    cols = int(z["cols"])
    assert _same_bits(gguf_ref.dequantize(qtype, z[f"raw_{qtype}"], cols), z[f"out_{qtype}"].view(np.float32))


@pytest.mark.skipif(not ref_lib.available(), reason="oracle/_ref not built (make -C oracle)")
@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_reference_build(qtype: str) -> None:
    """The numpy dequant equals the reference's compiled dequant_rows on fresh random tensors (the reference's
    test_dequant_rows: 33 x 1024, seed 1; tests/test_gguf_model.py:116-124)."""
    raw = tensors.random_blocks(qtype, 33, 1024, 1)
    assert _same_bits(gguf_ref.dequantize(qtype, raw, 1024), ref_lib.dequant_rows(qtype, raw, 1024))


def test_dequant_closed_forms() -> None:
    """Q4_0 nibble order and offset, Q8_0 sign, Q4_K 6-bit packing and min term, each on a hand-built block."""
    b = np.zeros((1, 18), np.uint8)
    b[0, :2] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1
    b[0, 2:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    w = gguf_ref.dequantize("Q4_0", b, 32)[0]
    assert w[:16].tolist() == [q - 8 for q in range(16)] and w[16:].tolist() == [q - 8 for q in range(15, -1, -1)]
    b = np.zeros((1, 34), np.uint8)
    b[0, :2] = np.array([0xB800], np.uint16).view(np.uint8)  # d = -0.5
    b[0, 2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert gguf_ref.dequantize("Q8_0", b, 32)[0].tolist() == [-0.5 * q for q in range(-16, 16)]
    b = np.zeros((1, 144), np.uint8)
    b[0, :4] = np.array([0x3C00, 0x3800], np.uint16).view(np.uint8)  # d = 1, dmin = 0.5
    sc = np.array([1, 2, 3, 4, 63, 62, 61, 60])
    mn = np.array([5, 6, 7, 8, 33, 34, 35, 36])
    s = b[0, 4:16]
    s[0:4] = (sc[:4] & 63) | ((sc[4:] >> 4) << 6)
    s[4:8] = (mn[:4] & 63) | ((mn[4:] >> 4) << 6)
    s[8:12] = (sc[4:] & 15) | ((mn[4:] & 15) << 4)
    b[0, 16:] = 0x21  # (low nibble 1, high nibble 2)
    f = gguf_ref.fields("Q4_K", b, 256)
    assert f["sc"][0, 0].tolist() == sc.tolist() and f["mn"][0, 0].tolist() == mn.tolist()
    w = gguf_ref.dequantize("Q4_K", b, 256)[0].reshape(8, 32)
    want = [(1 if g % 2 == 0 else 2) * sc[g] - 0.5 * mn[g] for g in range(8)]
    assert np.array_equal(w, np.repeat(np.array(want, np.float32)[:, None], 32, 1))


def _f16_bytes(*v: float) -> np.ndarray:
    return np.array(v, np.float16).view(np.uint8)


def test_dequant_closed_forms_more_types() -> None:
    """Q4_1's added min, Q5_K's fifth bit (bit g of qh[l]), Q6_K's crumb order, offset 32 and int8 sub-block scales,
    Q3_K's offset 4, high bit (hmask bit 4 n + j) and scales - 32, IQ4's table and IQ4_XS's 6-bit group scales, each on
    a hand-built block whose values the formats' layout fixes."""
    b = np.zeros((1, 20), np.uint8)
    b[0, :4] = _f16_bytes(2.0, -1.0)
    b[0, 4:] = np.arange(16, dtype=np.uint8) | (15 << 4)
    assert gguf_ref.dequantize("Q4_1", b, 32)[0].tolist() == [2.0 * q - 1 for q in range(16)] + [29.0] * 16
    b = np.zeros((1, 176), np.uint8)
    b[0, :4] = _f16_bytes(1.0, 0.0)
    b[0, 4:8] = 1  # groups 0..3: scale 1 (groups 4..7: 0)
    b[0, 16:48] = 0b00000010  # the fifth bit for group 1 only
    b[0, 48:] = 0x53  # group 0 (low nibble) 3, group 1 (high) 5 | 16
    w = gguf_ref.dequantize("Q5_K", b, 256)[0].reshape(8, 32)
    assert w[0].tolist() == [3.0] * 32 and w[1].tolist() == [21.0] * 32 and w[2:4].tolist() == [[3.0] * 32, [5.0] * 32]
    assert not w[4:].any()
    b = np.zeros((1, 210), np.uint8)
    b[0, 208:] = _f16_bytes(0.5)
    b[0, 192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)  # sub-block j: scale j - 8
    b[0, 0:128] = 0x21  # low nibble 1 (jj 0, 1), high nibble 2 (jj 2, 3)
    b[0, 128:192] = 0b11100100  # crumb jj = jj
    w = gguf_ref.dequantize("Q6_K", b, 256)[0].reshape(16, 16)
    want = [((1 if (j % 8) // 2 < 2 else 2) + 16 * ((j % 8) // 2) - 32) * 0.5 * (j - 8) for j in range(16)]
    assert np.array_equal(w, np.repeat(np.array(want, np.float32)[:, None], 16, 1))
    b = np.zeros((1, 110), np.uint8)
    b[0, 108:] = _f16_bytes(1.0)
    b[0, 96:104] = 0x21  # sub-blocks 0..7: low nibble 1, 8..15: 2 (no high crumbs): scales - 32
    b[0, 32:96] = 0b11100100  # crumb j = j
    b[0, 0:32] = 0x0F  # the high bit for n = 0 (bits 0..3), not for n = 1
    w = gguf_ref.dequantize("Q3_K", b, 256)[0].reshape(16, 16)  # sub-block 2 (4 n + j) + h
    want = [((j // 2) % 4 + (4 if j < 8 else 0) - 4) * ((1 if j < 8 else 2) - 32) for j in range(16)]
    assert np.array_equal(w, np.repeat(np.array(want, np.float32)[:, None], 16, 1))
    b = np.zeros((1, 18), np.uint8)
    b[0, :2] = _f16_bytes(1.0)
    b[0, 2:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    iq4 = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    assert gguf_ref.dequantize("IQ4_NL", b, 32)[0].tolist() == iq4 + iq4[::-1]
    b = np.zeros((1, 136), np.uint8)
    b[0, :2] = _f16_bytes(0.25)
    b[0, 2:4] = np.array([0b1110010011100100], np.uint16).view(np.uint8)  # crumb g = g % 4
    b[0, 4:8] = [0x10, 0x32, 0x54, 0x76]  # nibble g = g
    b[0, 8:] = 0x88  # code 8: IQ4 value 1
    w = gguf_ref.dequantize("IQ4_XS", b, 256)[0].reshape(8, 32)
    assert w.tolist() == [[0.25 * (g + 16 * (g % 4) - 32)] * 32 for g in range(8)]


def test_dequant_subnormal_scales() -> None:
    """fp16 subnormal scales are kept exactly: m 2^-24."""
    b = np.zeros((1, 18), np.uint8)
    b[0, :2] = np.array([0x0003], np.uint16).view(np.uint8)
    b[0, 2:] = 0xFF
    assert gguf_ref.dequantize("Q4_0", b, 32)[0].tolist() == [7 * 3 * 2.0 ** -24] * 32


# ---- the layer oracle's routing (tests/moe/ref.py:11-18) and the C++ host routing (moe_host.cpp:45-73)


def test_moe_route_known_answers() -> None:
    """The planted rows: equal maxima in id order, an all-equal row the lowest ids, +0 and -0 tied; int64 ids."""
    lg, planted = known_answers.planted_logits(1024)
    ids, w = moe_ref.moe_route(lg, 8)
    known_answers.assert_planted(ids, planted)
    assert np.allclose(w[1], 1 / 8) and ids.dtype == np.int64


def test_moe_route_brute_force() -> None:
    """Tiny rows against an exhaustive choice of the k-subset with the largest probabilities (ties to lower ids)."""
    rng = np.random.default_rng(3)
    lg = rng.integers(-3, 3, (200, 6)).astype(np.float32)  # (many ties)
    ids, w = moe_ref.moe_route(lg, 3)
    p = np_ops.softmax(lg)
    for t in range(lg.shape[0]):
        best = max(itertools.permutations(range(6), 3), key=lambda c: [(p[t, e], -e) for e in c])
        assert tuple(ids[t]) == best
        assert abs(w[t].sum() - 1) < 3e-7


def test_softmax_sum_in_float64() -> None:
    """softmax: the max subtracted; the sum in float64 (a float32 sum of 2^24 ones + extras would lose them)."""
    x = np.zeros((1, 4), np.float32)
    x[0, 0] = 1000.0  # (the max subtracted: no overflow)
    assert np.allclose(np_ops.softmax(x)[0], [1, 0, 0, 0])
    x = np.zeros((1, (1 << 24) + 4), np.float32)
    assert np_ops.softmax(x)[0, 0] == np.float32(1 / x.shape[1])


def test_row_sum_order() -> None:
    """numpy's pairwise order of moe_host.cpp:25-39: for 8 terms ((r0 + r1) + (r2 + r3)) + ..., not left to right;
    below 8 terms left to right."""
    e = np.array([[1.0, 1e16, -1e16, 1.0, 0, 0, 0, 0]])
    assert host_ref.row_sum(e)[0] == 0.0  # (left to right would give 1)
    assert host_ref.row_sum(e[:, :4])[0] == 1.0
    e = np.random.default_rng(1).random((50, 21))  # (21 terms: 8 sums over strides 0 and 8, then terms 16 .. 20)
    r = [e[:, j] + e[:, j + 8] for j in range(8)]
    s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
    for j in range(16, 21):
        s = s + e[:, j]
    assert np.array_equal(host_ref.row_sum(e), s)


def test_host_route_matches_oracle() -> None:
    """The reference's test_route: the C++ host routing (by logit) equals the oracle (by probability), weights within
    2e-7, from plain (T, E) rows and from the router GEMM's layout (32 experts per column at a pitch of 64, NaN in
    the gaps)."""
    lg, _ = known_answers.planted_logits(1024)
    rids, rw = moe_ref.moe_route(lg, 8)
    rows = known_answers.router_gemm_rows(lg)
    for args in ((lg.reshape(-1), 1024, 256, 256, 0, 256, 8), (rows.reshape(-1), 1024, 512, 32, 64, 256, 8)):
        ids, w = host_ref.moe_route(*args)
        assert np.array_equal(ids, rids) and ids.dtype == np.int32
        assert np.abs(w - rw).max() < 2e-7


def test_host_route_sigmoid_and_errors() -> None:
    """Sigmoid gating: sigmoid(l) over their sum, the sum clamped at 2^-14; the argument errors of moe_host.cpp:188."""
    lg = np.full((1, 4), -30.0, np.float32)
    ids, w = host_ref.moe_route(lg.reshape(-1), 1, 4, 4, 0, 4, 2, sigmoid=True)
    s = 1 / (1 + np.exp(30.0))
    assert ids.tolist() == [[0, 1]] and np.allclose(w, s / 2.0 ** -14)
    for k, E, pc in ((0, 4, 4), (5, 4, 4), (2, 6, 4)):
        with pytest.raises(host_ref.HostError):
            host_ref.moe_route(np.zeros(64, np.float32), 1, E, pc, 0, E, k)


def test_tie_collapse_detector() -> None:
    """Two distinct logits a float32 ulp apart can have equal fp32 probabilities: the detector flags them."""
    lg = np.zeros((1, 16), np.float32)
    lg[0, :] = -10.0
    lg[0, 3] = 1.0
    lg[0, 7] = np.nextafter(np.float32(1.0), np.float32(2.0))
    p = np_ops.softmax(lg)
    if p[0, 3] == p[0, 7]:
        assert layers.tie_collapsed(lg, 2)[0]
    assert not layers.tie_collapsed(np.arange(16, dtype=np.float32)[None], 2)[0]


# ---- the chunk plan (moe_host.cpp:201-235) and the dispatch under it


@pytest.mark.parametrize("T", [24, 2048])
def test_plan_invariants(T: int) -> None:
    """The reference test_plan's invariants on the oracle's plan of its routings."""
    from types import SimpleNamespace

    rng = np.random.default_rng(T)
    lg = rng.standard_normal((T, 256)).astype(np.float32) + np.linspace(0, 3, 256, dtype=np.float32)
    ids, _ = host_ref.moe_route(lg.reshape(-1), T, 256, 256, 0, 256, 8)
    cap = -(-(256 + -(-T * 8 // 192)) // 8)
    p = host_ref.moe_plan(ids, 256, 8, cap, 192)
    n = p["counts"]
    plan = SimpleNamespace(experts=[p["experts"][c, :n[c]] for c in range(8)], sizes=[p["sizes"][c, :n[c]] for c in range(8)],
                           rows=[p["rows"][c, :n[c]] for c in range(8)], pos=p["pos"], counts=n.tolist())
    known_answers.check_plan(plan, ids, cap)


def test_plan_errors() -> None:
    ids = np.array([[0, 1], [2, 3]], np.int32)
    with pytest.raises(host_ref.HostError, match="expert id 3 of 3"):
        host_ref.moe_plan(ids, 3, 8, 4, 192)
    with pytest.raises(host_ref.HostError, match="more than 0 chunks"):
        host_ref.moe_plan(ids, 4, 8, 0, 192)


def test_dispatch_brute_force() -> None:
    """Counts, offsets, order and slot against loops over the pairs (stable: pair order within an expert)."""
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 7, (40, 3))
    d = host_ref.dispatch(ids, 7)
    flat = ids.ravel().tolist()
    want = [p for e in range(7) for p in range(len(flat)) if flat[p] == e]
    assert d["order"].tolist() == want
    assert d["counts"].tolist() == [flat.count(e) for e in range(7)]
    assert d["offsets"][-1] == len(flat) and all(d["order"][d["slot"][p]] == p for p in range(len(flat)))


# ---- the layer oracle


def test_layer_oracle_f64_agreement() -> None:
    """The fp32 layer oracle is within 2e-6 relative L2 of the float64 one on the CPU configuration (same routing)."""
    spec = layers.CONFIGS["cpu"]
    layer = layers.make_layer(spec, 0)
    x = layers.make_x(spec, 16, 0)
    out = layers.forward(layer, x)
    y64 = layers.forward_f64(layer, x, out["ids"], out["w"])
    assert np.linalg.norm(out["y"] - y64) / np.linalg.norm(y64) < 2e-6


def test_layer_oracle_expert_loop() -> None:
    """moe_ffn sums each token's k expert outputs with its weights (a direct per-token loop agrees)."""
    spec = layers.CONFIGS["cpu"]
    layer = layers.make_layer(spec, 1)
    x = layers.make_x(spec, 5, 1)
    out = layers.forward(layer, x)
    get = layers.expert(layer)
    for t in range(5):
        y = sum(out["w"][t, i] * moe_ref.swiglu(x[t:t + 1], *get(int(out["ids"][t, i])))[0] for i in range(2))
        assert np.linalg.norm(out["y"][t] - y) / np.linalg.norm(y) < 1e-5


def test_zipf_config_routing() -> None:
    """Config 5's bias: about half the assignments on 4 hot experts, 6 experts with no token. (The router comes
    first from the layer's seed, so a layer of narrow experts has config 5's router and is quick to make.)"""
    spec = dataclasses.replace(layers.CONFIGS["skewed"], F=32)
    layer = layers.make_layer(spec, 0)
    x = layers.make_x(spec, 2048, 0)
    ids, _ = moe_ref.moe_route(layers.logits(layer, x), spec.k)
    c = np.bincount(ids.ravel(), minlength=spec.E)
    assert (c == 0).sum() == 6 and 0.4 < np.sort(c)[::-1][:4].sum() / c.sum() < 0.6


def test_rms_norm_pins() -> None:
    """rms_norm (tests/np_ops.py:27-32 restated): closed forms and a per-element float64 loop."""
    # a constant row c: c / sqrt(c^2 + eps), then times w
    for c in (3.0, -0.5, 1e-3):
        x = np.full((1, 64), c, np.float32)
        w = np.linspace(0.5, 1.5, 64).astype(np.float32)
        want = np.float32(np.float64(np.float32(c)) / np.sqrt(np.float64(np.float32(c)) ** 2 + 1e-6)) * w
        assert np.array_equal(np_ops.rms_norm(x, w, 1e-6), want[None])
    # zeros stay zeros; eps = 0 makes the row's RMS exactly 1 (up to one rounding)
    assert not np_ops.rms_norm(np.zeros((2, 8), np.float32), None, 1e-5).any()
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 96)).astype(np.float32) * 7
    y = np_ops.rms_norm(x, None, 0.0).astype(np.float64)
    assert np.allclose(np.sqrt((y ** 2).mean(1)), 1.0, rtol=1e-6)
    # per element: the float64 mean of squares, the quotient in float64 rounded once, then the fp32 product
    w = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    got = np_ops.rms_norm(x, w, 1e-6)
    for t in range(5):
        ms = sum(float(v) * float(v) for v in x[t].astype(np.float64)) / 96
        d = np.sqrt(ms + 1e-6)
        for i in range(96):
            assert got[t, i] == np.float32(np.float32(np.float64(x[t, i]) / d) * w[i])


# ---- closed-form pins of the fp32 ops and the layer formulas (tests/np_ops.py:10-17, tests/moe/ref.py:11-24,55-60):
# each case has an answer the mathematics fixes independently of the oracle's own formula, chosen so that swapping
# gate and up, taking silu for sigmoid, dropping the gate of the shared expert or transposing down fails


def _f32_close(got: object, want: float, ulps: int = 1) -> bool:
    g = np.float32(got)
    w = np.float32(want)
    return abs(int(np.array(g).view(np.int32)) - int(np.array(w).view(np.int32))) <= ulps


def test_sigmoid_closed_forms() -> None:
    """sigmoid(0) = 1/2 exactly; sigmoid(ln 3) = 3/4, sigmoid(-ln 3) = 1/4; sigmoid(x) + sigmoid(-x) = 1; the
    saturated ends exactly 0 and 1."""
    assert np_ops.sigmoid(np.float32(0.0)) == np.float32(0.5)
    ln3 = np.float32(np.log(3.0))
    assert _f32_close(np_ops.sigmoid(ln3), 0.75) and _f32_close(np_ops.sigmoid(-ln3), 0.25)
    x = np.linspace(-12, 12, 97, dtype=np.float32)
    assert np.abs(np_ops.sigmoid(x).astype(np.float64) + np_ops.sigmoid(-x) - 1).max() < 2 ** -23
    assert np_ops.sigmoid(np.float32(-100.0)) == 0.0 and np_ops.sigmoid(np.float32(100.0)) == 1.0
    assert np.all(np.diff(np_ops.sigmoid(x)) >= 0)  # (monotone)


def test_silu_closed_forms() -> None:
    """silu(0) = 0; silu(2) = 2 / (1 + e^-2) (not sigmoid(2)); silu(x) - silu(-x) = x; silu(x) = x for large x and -0
    for very negative x (e^-x overflows: x / inf); the minimum near x = -1.278 at about -0.2785."""
    assert np_ops.silu(np.float32(0.0)) == 0.0
    assert _f32_close(np_ops.silu(np.float32(2.0)), 2.0 / (1.0 + np.exp(-2.0)))
    assert not _f32_close(np_ops.silu(np.float32(2.0)), 1.0 / (1.0 + np.exp(-2.0)), 1000)
    x = np.linspace(-9, 9, 73, dtype=np.float32)
    assert np.abs(np_ops.silu(x).astype(np.float64) - np_ops.silu(-x) - x).max() < 4e-6
    assert np_ops.silu(np.float32(30.0)) == np.float32(30.0)
    r = np_ops.silu(np.float32(-100.0))
    assert r == 0.0 and np.signbit(r)
    t = np.linspace(-3, 0, 3001, dtype=np.float32)
    assert abs(float(np_ops.silu(t).min()) + 0.27846) < 1e-4 and abs(float(t[np_ops.silu(t).argmin()]) + 1.2785) < 2e-3


def test_swiglu_closed_form() -> None:
    """A one-hot FFN (H = 3, F = 2): gate row 0 picks x0, up row 0 picks 2 x1, down column 0 lands in output 2, so
    y = [0, 0, silu(x0) 2 x1] exactly up to fp32 rounding; swapping gate and up would give silu(2 x1) x0."""
    gate = np.array([[1, 0, 0], [0, 0, 0]], np.float32)
    up = np.array([[0, 2, 0], [0, 0, 0]], np.float32)
    down = np.zeros((3, 2), np.float32)
    down[2, 0] = 1.0
    x = np.array([[2.0, 3.0, 5.0], [-1.0, 0.5, 7.0]], np.float32)
    y = moe_ref.swiglu(x, gate, up, down)
    for t in range(2):
        x0, x1 = float(x[t, 0]), float(x[t, 1])
        want = x0 / (1 + np.exp(-x0)) * 2 * x1
        assert y[t, 0] == 0 and y[t, 1] == 0 and _f32_close(y[t, 2], want, 2)
        assert not _f32_close(y[t, 2], 2 * x1 / (1 + np.exp(-2 * x1)) * x0, 1000)
    # a diagonal FFN: y_i = silu(a_i x_i) b_i x_i c_i for diagonal gate a, up b, down c
    a, b, c = (np.array(v, np.float32) for v in ([0.5, -2.0, 1.5], [3.0, 0.25, -1.0], [2.0, 1.0, -0.5]))
    x = np.array([[1.0, 2.0, -3.0]], np.float32)
    y = moe_ref.swiglu(x, np.diag(a), np.diag(b), np.diag(c))[0]
    for i in range(3):
        g = float(a[i] * x[0, i])
        assert _f32_close(y[i], g / (1 + np.exp(-g)) * float(b[i] * x[0, i]) * float(c[i]), 3)


def test_shared_expert_gate() -> None:
    """The shared expert: without gate_inp exactly swiglu(x); with a gate_inp orthogonal to x, sigmoid(0) = 1/2, so
    exactly half of it; with x . gate_inp = ln 3, three quarters."""
    rng = np.random.default_rng(4)
    H, F = 8, 6
    g, u = rng.standard_normal((F, H)).astype(np.float32), rng.standard_normal((F, H)).astype(np.float32)
    d = rng.standard_normal((H, F)).astype(np.float32)
    x = np.zeros((2, H), np.float32)
    x[0, :4] = [1.0, -2.0, 0.5, 3.0]
    x[1, 4:] = [0.25, 1.0, -1.0, 2.0]
    full = moe_ref.swiglu(x, g, u, d)
    assert np.array_equal(moe_ref.shared_expert(x, g, u, d, None), full)
    gi = np.zeros(H, np.float32)  # x0 . gi = 1 (-1) + 0.5 (2) = 0; x1 has nothing at 0 or 2
    gi[2] = 2.0
    gi[0] = -1.0
    assert np.array_equal(moe_ref.shared_expert(x, g, u, d, gi), np.float32(0.5) * full)
    gi = np.zeros(H, np.float32)
    gi[3] = np.float32(np.log(3.0)) / np.float32(3.0)  # (x0 . gi = ln 3)
    s = moe_ref.shared_expert(x, g, u, d, gi)
    assert np.allclose(s[0], 0.75 * full[0], rtol=2e-7, atol=0) and np.array_equal(s[1], 0.5 * full[1])


def test_moe_route_closed_forms() -> None:
    """Softmax gating: logits ln(1, 2, 3, 4) have p = (0.1, 0.2, 0.3, 0.4), so top 2 is (3, 2) with weights 4/7, 3/7.
    Sigmoid gating: logits (0, ln 3, -ln 3, 2) have sigmoids (1/2, 3/4, 1/4, 0.8808), so top 2 is (3, 1) with weights
    s3 / (s3 + 3/4) and 3/4 / (s3 + 3/4); ties to the lower id; a sum below 2^-14 is clamped to it."""
    lg = np.log(np.array([[1.0, 2.0, 3.0, 4.0]])).astype(np.float32)
    ids, w = moe_ref.moe_route(lg, 2)
    assert ids.tolist() == [[3, 2]] and _f32_close(w[0, 0], 4 / 7, 2) and _f32_close(w[0, 1], 3 / 7, 2)
    ln3 = float(np.float32(np.log(3.0)))
    lg = np.array([[0.0, ln3, -ln3, 2.0], [1.0, 1.0, 1.0, -1.0], [-30.0, -30.0, -31.0, -32.0]], np.float32)
    ids, w = moe_ref.moe_route(lg, 2, gating="sigmoid")
    s3 = 1 / (1 + np.exp(-2.0))
    assert ids[0].tolist() == [3, 1]
    assert _f32_close(w[0, 0], s3 / (s3 + 0.75), 2) and _f32_close(w[0, 1], 0.75 / (s3 + 0.75), 2)
    assert ids[1].tolist() == [0, 1] and w[1, 0] == w[1, 1] == np.float32(0.5)
    tiny = 1 / (1 + np.exp(30.0))
    assert ids[2].tolist() == [0, 1] and _f32_close(w[2, 0], tiny / 2.0 ** -14, 4)  # (the clamp, not 1/2)
    with pytest.raises(AssertionError):
        assert _f32_close(w[2, 0], 0.5, 1000)


def test_router_logits_closed_form() -> None:
    """The router logits x W^T (float64, one rounding): a one-hot token picks a router column exactly; a token of
    2^-j weights sums exactly representable terms, the float64 sum then rounded once."""
    spec = layers.CONFIGS["cpu"]
    layer = layers.make_layer(spec, 0)
    x = np.zeros((2, spec.H), np.float32)
    x[0, 17] = 1.0
    x[1, :3] = [0.5, 0.25, -2.0]
    lg = layers.logits(layer, x)
    assert np.array_equal(lg[0], layer.router[:, 17])
    r = layer.router.astype(np.float64)
    assert np.array_equal(lg[1], (0.5 * r[:, 0] + 0.25 * r[:, 1] - 2.0 * r[:, 2]).astype(np.float32))
