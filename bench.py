"""The headline benchmark: MoE-layer tokens/s of a Qwen3-30B-A3B-shaped Q4_0 layer (H 2048, 128 experts, top 8,
SwiGLU F 768) on one MI355X, at decode (16 tokens: ``value``) and at a 4096-token prefill (``prefill``), with the
dominant kernel's roofline fraction and the numpy CPU oracle timed on the host beside it.

One step = one layer forward (router, routing, dispatch, experts, combine) over one batch already resident in HBM.
Steps cycle through ``--weight-sets`` distinct weight sets so the decode working set (~220 MB per call) streams from
HBM rather than the 256 MB Infinity Cache. Timing uses HIP events on the layer's stream (``artlite_moe_layer_time``).
Prints ONE JSON line."""

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA, TFLOP/s
METRIC = "MoE-layer tok/s at decode B=16 and prefill 4096; % of HBM / MFMA roofline"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


BLOCK = {"Q4_0": (32, 18, (0,)), "Q8_0": (32, 34, (0,)), "Q4_K": (256, 144, (0, 2))}


def synth_blocks(rng: np.random.Generator, qtype: str, rows: int, cols: int, scale: float) -> np.ndarray:
    """Random GGUF blocks: bytes uniform, fp16 scales |N(0, scale)| (BASELINE configurations 2 and 3)."""
    per, nb, f16 = BLOCK[qtype]
    raw = rng.integers(0, 256, (rows, cols // per, nb), dtype=np.uint8)
    for o in f16:
        d = np.abs(rng.standard_normal((rows, cols // per)) * scale).astype(np.float16)
        raw[..., o:o + 2] = d.view(np.uint8).reshape(rows, cols // per, 2)
    return raw.reshape(rows, -1)


def synth_layer(shape: dict, seed: int) -> dict:
    """A Qwen3-30B-A3B-shaped layer: router fp32 N(0, 0.02) (prefill: U(-0.035, 0.035)), Q4_0 experts."""
    rng = np.random.default_rng(seed)
    H, E, F, q = shape["H"], shape["E"], shape["F"], shape["qtype"]
    if shape["router"] == "uniform":
        router = rng.uniform(-0.035, 0.035, (E, H)).astype(np.float32)
    else:
        router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    return {"ffn_gate_inp": router, "ffn_gate_exps": synth_blocks(rng, q, E * F, H, 0.02),
            "ffn_up_exps": synth_blocks(rng, q, E * F, H, 0.02), "ffn_down_exps": synth_blocks(rng, q, E * H, F, 0.02)}


def synth_x(H: int, T: int, seed: int) -> np.ndarray:
    """bf16 activations N(0, 1) as bit patterns (round to nearest even)."""
    x = np.random.default_rng(10_000 + seed).standard_normal((T, H)).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def measure(shape: dict, T: int, n_sets: int, steps: int, warmup: int) -> dict:
    from artlite_amd.moe.layer import MoELayer, time_layers

    gls = []
    for i in range(n_sets):
        g = MoELayer(hidden=shape["H"], n_experts=shape["E"], top_k=shape["k"], expert_ffn=shape["F"],
                     gate_type=shape["qtype"], down_type=shape["qtype"], max_tokens=T)
        for name, a in synth_layer(shape, 100 + i).items():
            g.upload(name, a)
        gls.append(g)
        log(f"weight set {i + 1}/{n_sets} uploaded")
    x = synth_x(shape["H"], T, 0)
    U = []
    for g in gls:
        g(x)  # (a run: the experts touched, and a warm start)
        U.append(int((g.tap("counts") > 0).sum()))
        g.stage(x)
    ms, per_kernel = time_layers(gls, warmup=warmup, iters=steps)
    for g in gls:
        g.close()
    return {"ms": ms, "kernels": per_kernel, "U": float(np.mean(U))}


def bpw(qtype: str) -> float:
    return {"Q4_0": 18 / 32, "Q8_0": 34 / 32, "Q4_K": 144 / 256}[qtype]


def cpu_baseline(shape: dict, T: int, budget_s: float) -> dict:
    """The numpy oracle (router in float64, routing, per-expert dequantization, fp32 SwiGLU) on the same workload (the
    first weight set, the same tokens), single-threaded BLAS, repeated for about ``budget_s`` seconds."""
    from threadpoolctl import threadpool_limits

    from oracle import layers
    from oracle.tensors import from_bf16_bits

    spec = layers.CONFIGS["decode"]
    w = synth_layer(shape, 100)
    layer = layers.Layer(spec, w["ffn_gate_inp"], w["ffn_gate_exps"], w["ffn_up_exps"], w["ffn_down_exps"])
    x = from_bf16_bits(synth_x(shape["H"], T, 0))
    times = []
    with threadpool_limits(1):
        t_end = time.perf_counter() + budget_s
        while not times or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            layers.forward(layer, x)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": T / med, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} full layer calls of {T} tokens (numpy oracle, 1 BLAS thread), median "
                      f"{med * 1e3:.0f} ms; host {os.cpu_count()} logical CPUs"}


def traffic_bytes(path: str) -> float | None:
    """HBM bytes per launch of the decode gate / up kernel from its counter summary (the line
    ``traffic_bytes_per_launch: N``: FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the copy calibration), or
    None without one."""
    try:
        for line in Path(path).read_text().splitlines():
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=16)
    ap.add_argument("--weight-sets", type=int, default=4)
    ap.add_argument("--prefill-tokens", type=int, default=4096)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (the calibration kernel of counter profiles)")
    ap.add_argument("--traffic", default=str(ROOT / "profiles" / "gemv_gate_up_decode_b16_traffic.md"),
                    help="the counter summary giving the decode gate / up kernel's HBM bytes per launch")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU (asked for {args.gpus}); the path is single-GPU by design",
              file=sys.stderr)
        sys.exit(2)

    from artlite_amd import device_count

    assert device_count() > 0, "no GPU visible"
    shape = {"H": 2048, "E": 128, "k": 8, "F": 768, "qtype": "Q4_0", "router": "normal"}
    H, F, E, k = shape["H"], shape["F"], shape["E"], shape["k"]
    T = args.tokens
    log(f"decode: T={T}, {args.weight_sets} weight sets")
    dec = measure(shape, T, args.weight_sets, args.steps, args.warmup)
    if args.copy_probe:
        from artlite_amd.moe.layer import hbm_copy_ms

        log(f"copy probe: {args.copy_probe} MiB, {hbm_copy_ms(args.copy_probe << 20, 1):.3f} ms")
    ms = dec["ms"]
    U = dec["U"]
    # algorithmic bytes: the layer (weights of the experts touched, router, x in, y out) and the dominant kernel
    # (gate / up: its weights and x)
    layer_bytes = U * 3 * H * F * bpw(shape["qtype"]) + E * H * 4 + T * H * 2 + T * H * 4
    gu_bytes = U * 2 * H * F * bpw(shape["qtype"]) + T * H * 2
    gu_ms = dec["kernels"].get("gate_up", float("nan"))
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "i8", "data": "synthetic",
        "config": {"workload": "qwen3-30b-a3b-shaped MoE layer, Q4_0 experts, decode", "tokens": T, "hidden": H,
                   "experts": E, "top_k": k, "expert_ffn": F, "weights": shape["qtype"], "activations": "bf16",
                   "weight_sets": args.weight_sets, "experts_touched": U},
        "roofline": {"bound": "hbm", "kernel": "gate_up", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_bytes(args.traffic), "kernel_ms": gu_ms,
                     "algorithmic_bytes": gu_bytes},
        "layer_roofline": {"bound": "hbm", "achieved": layer_bytes / (ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                           "algorithmic_bytes": layer_bytes},
        "kernel_ms": dec["kernels"],
    }
    if not args.no_prefill:
        Tp = args.prefill_tokens
        log(f"prefill: T={Tp}")
        pre = measure({**shape, "router": "uniform"}, Tp, 1, args.prefill_steps, 2)
        flops = 2 * Tp * k * 3 * H * F + 2 * Tp * H * E
        gu_flops = 2 * Tp * k * 2 * H * F
        pgu = pre["kernels"].get("gate_up", float("nan"))
        out["prefill"] = {"tokens": Tp, "value": Tp / (pre["ms"] * 1e-3), "unit": "tokens/s", "ms_per_step": pre["ms"],
                          "dtype": "f16",
                          "steps": args.prefill_steps, "kernel_ms": pre["kernels"],
                          "roofline": {"bound": "mfma", "kernel": "gate_up", "achieved": gu_flops / (pgu * 1e-3) / 1e12,
                                       "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                       "frac": gu_flops / (pgu * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                                       "traffic": None},
                          "layer_roofline": {"bound": "mfma", "achieved": flops / (pre["ms"] * 1e-3) / 1e12,
                                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                             "frac": flops / (pre["ms"] * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS}}
    if args.cpu_seconds > 0:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(shape, T, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
