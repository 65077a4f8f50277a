"""The GPU MoE layer against the oracle at the benchmark configurations' stated sizes (4, 5 and a
Q4_0 case whose experts all hold more than 64 rows), the way the reference checks a whole MoE block at its real
chunk size (``tests/moe/test_prefill.py:287-405``):

- router logits within one ulp (float64 accumulation on both sides); ids bit-exact against the C++ host routing's
  restatement of the GPU's logits and equal to the layer oracle's own routing except at near ties; counts, offsets,
  sorted order and slots bit-exact against the stable counting sort;
- h and every pair's expert output against float64 math for a sample of experts that includes the busiest and the
  least busy one (so the prefill tiles' 8-row-block form, which every expert with more than 64 rows takes, is
  covered);
- the layer output within 1e-3 relative L2 of the full fp32 oracle (``moe_ffn`` over every touched expert, plus the
  shared expert), and bitwise identical on a second run."""

import numpy as np
import pytest

from oracle import layers

from .helpers import check_against_oracle, check_pairs_f64, gpu_input, gpu_layer

pytestmark = pytest.mark.gpu


def run_full(name: str, T: int, seed: int = 0, plant=None) -> dict:
    spec = layers.CONFIGS[name]
    print(f"full-size layer {name} T={T} seed={seed}{' planted' if plant else ''}", flush=True)
    layer = layers.make_layer(spec, seed)
    if plant:
        plant(layer)
    x = layers.make_x(spec, T, seed)
    with gpu_layer(layer, max_tokens=T) as g:
        y = g(gpu_input(spec, x))
        kernels = g.kernel_names()
        taps = check_against_oracle(g, layer, x, y)
        counts, offsets, order = taps["counts"], taps["offsets"], taps["order"]
        busy = [int(np.argmax(counts)), int(np.argmin(np.where(counts > 0, counts, 1 << 30)))]
        rest = [e for e in np.random.default_rng(seed).permutation(spec.E).tolist() if e not in busy and counts[e]]
        check_pairs_f64(g, layer, x, offsets, order, busy + rest[:4], 1e-3)
        again = g(gpu_input(spec, x))
        assert np.array_equal(again.view(np.uint32), y.view(np.uint32)), "not deterministic"
    return {"kernels": kernels, "counts": counts, "rel_l2": taps["rel_l2"], "layer": layer}


def test_full_prefill_cfg3() -> None:
    """Config 3: the Qwen3-30B-A3B-shaped Q4_0 layer at 4096 tokens (uniform router): every expert holds more than 64
    of the 32768 pairs, so both prefill launches run their 8-row-block form for every tile but the last of each."""
    r = run_full("prefill", 4096)
    assert "prefill_x" in r["kernels"]
    assert r["counts"].min() > 64 and r["counts"].sum() == 4096 * 8


def test_full_deepseek_cfg4() -> None:
    """Config 4: the DeepSeek-V2-Lite-shaped layer (Q4_K gate / up, Q8_0 down, a Q4_K shared expert of 2816) at 512
    tokens, 64 experts top 6."""
    r = run_full("deepseek", 512)
    assert r["counts"].sum() == 512 * 6 and (r["counts"] > 0).sum() == 64
    # (the shared gate / up's items in the routed gate / up launch; its Q4_K down, unlike the routed Q8_0 one, in a
    # launch of its own over four parts of its K)
    assert "shared_gate_up" not in r["kernels"] and "shared_down" in r["kernels"], r["kernels"]


def test_full_skewed_cfg5() -> None:
    """Config 5: Zipf-skewed routing over 32 Q8_0 experts (H = F = 2880) at 2048 tokens: the 6 cold experts get no
    pair (empty groups), about half the pairs land on 4 hot ones."""
    r = run_full("skewed", 2048)
    c = r["counts"]
    assert (c == 0).sum() == 6 and np.array_equal(np.flatnonzero(c == 0), r["layer"].meta["cold"])
    assert 0.4 < np.sort(c)[::-1][:4].sum() / c.sum() < 0.6
    assert "prefill_x" in r["kernels"]


def plant_q8_outliers(layer: layers.Layer, factor: float = 32.0) -> None:
    """Multiply the fp16 scale of one Q8_0 block by ``factor`` in a row of the gate, the up and the down matrix of
    one routed expert that receives tokens (an outlier block, as real GGUF tensors hold them)."""
    spec = layer.spec
    e = next(i for i in range(spec.E) if i not in set(layer.meta.get("cold", [])))
    for m, row, blk in ((layer.gate, e * spec.F + 5, 3), (layer.up, e * spec.F + 9, 1), (layer.down, e * spec.H + 7, 2)):
        d = m[row, 34 * blk:34 * blk + 2].view(np.float16)
        m[row, 34 * blk:34 * blk + 2] = (d.astype(np.float32) * factor).astype(np.float16).view(np.uint8)


def test_full_skewed_outlier_scales() -> None:
    """Config 5 with one block of 32x the usual scale in a gate, an up and a down row of one routed expert: the prefill
    tiles' fp16 h and pair outputs take their scales from the matrices' largest row L1 norms (an outlier block raises
    one row's norm by its 32 values' share), so the layer stays within 1e-3 of the fp32 oracle and h and the pair
    outputs within 1e-3 of float64 math."""
    r = run_full("skewed", 2048, plant=plant_q8_outliers)
    assert "prefill_x" in r["kernels"]


def test_full_q4_rows() -> None:
    """A small Q4_0 layer (E = 8, top 2) at 512 tokens: about 128 rows per expert, the prefill tiles' 8-row-block form
    for Q4_0 in both launches."""
    r = run_full("q4_rows", 512)
    assert "prefill_x" in r["kernels"] and r["counts"].min() > 64


def test_full_k4_rows() -> None:
    """The same small layer in Q4_K (gate / up and down): the prefill tiles' super-block staging (headers and code
    quarters) and in-register decode in both launches, every expert over 64 rows."""
    r = run_full("k4_rows", 512)
    assert "prefill_x" in r["kernels"] and r["counts"].min() > 64


def test_full_q4km_prefill() -> None:
    """The Qwen3-30B-A3B shape as Q4_K_M files quantise it (Q4_K gate / up, Q6_K down) at 4096 tokens: gate / up on
    the prefill tiles from the file's Q4_K bytes, the down on the prefill tiles through the prefill layout of its Q6_K
    blocks (made at upload); every expert over 64 rows."""
    r = run_full("q4km", 4096)
    assert "prefill_x" in r["kernels"] and r["counts"].min() > 64 and r["counts"].sum() == 4096 * 8


def test_full_decode_cfg2_t64() -> None:
    """Config 2 at its largest decode batch (64 tokens) with a second seed."""
    r = run_full("decode", 64, seed=7)
    assert r["counts"].sum() == 64 * 8
