"""Pins the CPU oracle before anything is checked against it: against the reference's own compiled dequantizer and
its outputs committed under tests/golden, the known answers of the reference's tests (tests/moe/test_route.py,
tests/moe/test_plan.py), closed forms, brute force on tiny inputs, and properties chosen so that a plausible slip (a
dropped offset, a swapped nibble half, a sequential instead of pairwise sum, an unstable sort) fails."""

import itertools
from pathlib import Path

import numpy as np
import pytest

from oracle import gguf_ref, host_ref, layers, moe_ref, np_ops, ref_lib, tensors

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


def _test_route_logits() -> np.ndarray:
    """The logits of the reference's test_route (tests/moe/test_plan.py:18-33): ties at the top, all tied, -0 / +0."""
    rng = np.random.default_rng(0)
    lg = rng.standard_normal((1024, 256)).astype(np.float32) * 2
    lg[0, [3, 9, 200]] = lg[0].max() + 1
    lg[1, :] = 0.5
    lg[2, :8], lg[2, 8:] = -0.0, -1
    lg[2, 5] = 0.0
    return lg


def test_moe_route_known_answers() -> None:
    """The reference tests' known answers: a three-way tie at the top in id order, all-tied rows the lowest ids,
    -0 and +0 tied."""
    ids, w = moe_ref.moe_route(_test_route_logits(), 8)
    assert ids[0, :3].tolist() == [3, 9, 200] and ids[1].tolist() == ids[2].tolist() == list(range(8))
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
    lg = _test_route_logits()
    rids, rw = moe_ref.moe_route(lg, 8)
    rows = np.full((1024, 8, 64), np.nan, np.float32)
    rows[:, :, :32] = lg.reshape(1024, 8, 32)
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
    """The reference's test_plan (tests/moe/test_plan.py:36-67) on the oracle's plan."""
    rng = np.random.default_rng(T)
    lg = rng.standard_normal((T, 256)).astype(np.float32) + np.linspace(0, 3, 256, dtype=np.float32)
    ids, _ = host_ref.moe_route(lg.reshape(-1), T, 256, 256, 0, 256, 8)
    chunk, cols = 192, 8
    cap = -(-(256 + -(-T * 8 // chunk)) // cols)
    p = host_ref.moe_plan(ids, 256, cols, cap, chunk)
    counts = p["counts"]
    assert max(counts) - min(counts) <= 1
    assert sum(counts) == sum(-(-r // chunk) for r in np.bincount(ids.ravel()))
    g, j = np.divmod(p["pos"], chunk)
    c, k = np.divmod(g, cap)
    assert len(set(p["pos"].ravel().tolist())) == ids.size
    for t in range(T):
        for i in range(8):
            assert p["experts"][c[t, i], k[t, i]] == ids[t, i] and p["rows"][c[t, i], k[t, i], j[t, i]] == t
    for col in range(cols):
        for kk in range(counts[col]):
            r = p["rows"][col, kk]
            n = int(((c == col) & (k == kk)).sum())
            assert (r[n:] == r[0]).all() and (np.diff(r[:n]) > 0).all()


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
    """Config 5's bias: about half the assignments on 4 hot experts, 6 experts with no token."""
    spec = layers.CONFIGS["skewed"]
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
