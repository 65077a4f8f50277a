"""The headline benchmark: MoE-layer tokens/s of a Qwen3-30B-A3B-shaped Q4_0 layer (H 2048, 128 experts, top 8,
SwiGLU F 768) on one MI355X, at decode (16 tokens: ``value``) and at a 4096-token prefill (``prefill``), plus the
other BASELINE workloads (decode at 1, 4 and 64 tokens, and at 128, between decode and prefill sizes; the
DeepSeek-V2-Lite-shaped Q4_K layer at 512 tokens; the Zipf-skewed Q8_0 layer at 2048 tokens) and the prefill shape
with Q4_K gate / up and a Q6_K down (``q4km``, as Q4_K_M files hold it), each with its dominant kernel's roofline
fraction and the numpy CPU oracle timed on the host beside it.

One step = one layer forward (router, routing, dispatch, experts, combine) over one batch already resident in HBM.
Decode steps cycle through ``--weight-sets`` distinct weight sets so the working set (~220 MB per call) streams from
HBM rather than the 256 MB Infinity Cache. Timing uses HIP events on the layer's stream (``artlite_moe_layer_time``):
``ms_per_step`` is a timed region of back-to-back steps over the step count (events only at its ends, a
synchronization before it), ``ms_median_evented`` the median step of a second region with an event before each step
(each such event holds the step after it back by a few microseconds). Prints ONE JSON line."""

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 MFMA, TFLOP/s
METRIC = "MoE-layer tok/s at decode B=16 and prefill 4096; % of HBM / MFMA roofline"

# the BASELINE workloads (configs 2-5): shapes, formats, weight statistics
SHAPES = {
    "decode": dict(H=2048, E=128, k=8, F=768, gate="Q4_0", down="Q4_0", scale=0.02, router="normal"),
    "prefill": dict(H=2048, E=128, k=8, F=768, gate="Q4_0", down="Q4_0", scale=0.02, router="uniform"),
    "deepseek": dict(H=2048, E=64, k=6, F=1408, gate="Q4_K", down="Q8_0", scale=2e-4, dmin=1.5e-3, shared_F=2816,
                     shared="Q4_K", router="normal"),
    "skewed": dict(H=2880, E=32, k=4, F=2880, gate="Q8_0", down="Q8_0", scale=0.01, router="zipf"),
    # config 3's shape as Q4_K_M files quantise it (Q4_K gate / up, Q6_K down: the down through the prefill layout)
    "q4km": dict(H=2048, E=128, k=8, F=768, gate="Q4_K", down="Q6_K", scale=2e-4, dmin=1.5e-3, router="uniform"),
}
ZIPF_S, ZIPF_ACTIVE, ZIPF_BETA = 1.2, 26, 0.7  # config 5: 26 experts ranked by Zipf s = 1.2, 6 never chosen


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# (values per block, bytes per block, offsets of the fp16 fields: scale, then Q4_K's dmin)
BLOCK = {"Q4_0": (32, 18, (0,)), "Q8_0": (32, 34, (0,)), "Q4_K": (256, 144, (0, 2)), "Q6_K": (256, 210, (208,))}


def bpw(qtype: str) -> float:
    per, nb, _ = BLOCK[qtype]
    return nb / per


def synth_blocks(rng: np.random.Generator, qtype: str, rows: int, cols: int, scale: float,
                 dmin: float = 0.0) -> np.ndarray:
    """Random GGUF blocks: bytes uniform, fp16 scale |N(0, scale)| (Q4_K: dmin |N(0, dmin)|)."""
    per, nb, f16 = BLOCK[qtype]
    raw = rng.integers(0, 256, (rows, cols // per, nb), dtype=np.uint8)
    for i, o in enumerate(f16):
        d = np.abs(rng.standard_normal((rows, cols // per)) * (dmin if i else scale)).astype(np.float16)
        raw[..., o:o + 2] = d.view(np.uint8).reshape(rows, cols // per, 2)
    return raw.reshape(rows, -1)


def synth_layer(shape: dict, seed: int) -> dict:
    """A layer of ``shape``: router fp32 N(0, 0.02) (``uniform``: U(-0.035, 0.035); ``zipf``: plus a bias in column
    0, which the inputs' feature 0 = 1 adds to the logits), expert blocks (and a shared expert) of ``synth_blocks``."""
    rng = np.random.default_rng(seed)
    H, E, F = shape["H"], shape["E"], shape["F"]
    if shape["router"] == "uniform":
        router = rng.uniform(-0.035, 0.035, (E, H)).astype(np.float32)
    else:
        router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    if shape["router"] == "zipf":
        bias = np.full(E, -1e4, np.float64)
        hot = np.random.default_rng(seed + 1).permutation(E)[:ZIPF_ACTIVE]
        bias[hot] = ZIPF_BETA * -ZIPF_S * np.log(np.arange(1, ZIPF_ACTIVE + 1))
        router[:, 0] = bias.astype(np.float32)
    sc, dm = shape["scale"], shape.get("dmin", 0.0)
    w = {"ffn_gate_inp": router, "ffn_gate_exps": synth_blocks(rng, shape["gate"], E * F, H, sc, dm),
         "ffn_up_exps": synth_blocks(rng, shape["gate"], E * F, H, sc, dm),
         "ffn_down_exps": synth_blocks(rng, shape["down"], E * H, F, sc, dm)}
    if shape.get("shared_F"):
        Fs, st = shape["shared_F"], shape["shared"]
        w["ffn_gate_shexp"] = synth_blocks(rng, st, Fs, H, sc, dm)
        w["ffn_up_shexp"] = synth_blocks(rng, st, Fs, H, sc, dm)
        w["ffn_down_shexp"] = synth_blocks(rng, st, H, Fs, sc, dm)
    return w


def synth_x(shape: dict, T: int, seed: int = 0) -> np.ndarray:
    """bf16 activations N(0, 1) as bit patterns (round to nearest even); ``zipf``: feature 0 the constant 1."""
    x = np.random.default_rng(10_000 + seed).standard_normal((T, shape["H"])).astype(np.float32)
    if shape["router"] == "zipf":
        x[:, 0] = 1.0
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def build_layers(shape: dict, n_sets: int, max_T: int) -> list:
    from artlite_amd.moe.layer import MoELayer

    out = []
    for i in range(n_sets):
        g = MoELayer(hidden=shape["H"], n_experts=shape["E"], top_k=shape["k"], expert_ffn=shape["F"],
                     gate_type=shape["gate"], down_type=shape["down"], max_tokens=max_T,
                     shared_ffn=shape.get("shared_F", 0), shared_type=shape.get("shared", ""))
        for name, a in synth_layer(shape, 100 + i).items():
            g.upload(name, a)
        out.append(g)
        log(f"  weight set {i + 1}/{n_sets} uploaded")
    return out


def time_T(gls: list, shape: dict, T: int, steps: int, warmup: int) -> dict:
    """Steps of T tokens over the layers (one run first: the experts each touches); median and mean ms, per-kernel
    mean ms."""
    from artlite_amd.moe.layer import time_layers

    x = synth_x(shape, T)
    U = []
    for g in gls:
        g(x)
        U.append(int((g.tap("counts") > 0).sum()))
        g.stage(x)
    mean, runs, kernels = time_layers(gls, warmup=warmup, iters=steps)
    return {"ms": mean, "ms_median_evented": float(np.median(runs)), "kernels": kernels, "U": float(np.mean(U)),
            "names": list(kernels)}


def work(shape: dict, T: int, U: float, pair_bytes: int, names: list) -> dict:
    """Algorithmic bytes and flops of the layer and of its gate / up and down launches (U experts touched): the
    weights of the touched experts once, the activations in bf16, h in fp16, the pair outputs in ``pair_bytes`` per
    value (the path's format: fp16 on the prefill tiles, fp32 elsewhere), the layer's output in fp32. On the prefill
    tiles the shared expert's products join the routed launches of their format (``names`` then lacks
    ``shared_gate_up`` / ``shared_down``), and their work counts in those launches'."""
    H, E, k, F = shape["H"], shape["E"], shape["k"], shape["F"]
    P = T * k
    Fs = shape.get("shared_F", 0)
    gu_b = U * 2 * H * F * bpw(shape["gate"]) + T * H * 2
    dn_b = U * H * F * bpw(shape["down"]) + P * F * 2 + P * H * pair_bytes
    sh_b = 2 * H * Fs * bpw(shape["shared"]) + H * Fs * bpw(shape["shared"]) if Fs else 0.0
    layer_b = gu_b + dn_b + sh_b + E * H * 4 + T * H * 4
    gu_f = 2.0 * P * 2 * H * F
    dn_f = 2.0 * P * H * F
    if Fs and "prefill_x" in names:
        if "shared_gate_up" not in names:
            gu_b += 2 * H * Fs * bpw(shape["shared"]) + T * Fs * 2
            gu_f += 2.0 * T * 2 * H * Fs
        if "shared_down" not in names:
            dn_b += H * Fs * bpw(shape["shared"]) + T * Fs * 2 + T * H * 4
            dn_f += 2.0 * T * H * Fs
    layer_f = 2.0 * P * 3 * H * F + 2.0 * T * 3 * H * Fs + 2.0 * T * H * E
    return {"gate_up": (gu_b, gu_f), "down": (dn_b, dn_f), "layer": (layer_b, layer_f)}


def traffic(path: Path, kernel: str) -> tuple[float | None, str | None]:
    """(HBM bytes per launch, where from) of a kernel in a counter summary under profiles/: its line
    ``traffic_bytes_per_launch[kernel]: N`` (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the copy
    calibration) and the summary's ``commit:`` line."""
    try:
        lines = path.read_text().splitlines()
    except OSError:
        return None, None
    val, commit = None, "?"
    for line in lines:
        s = line.strip().lstrip("-* ")
        if s.startswith(f"traffic_bytes_per_launch[{kernel}]:"):
            val = float(s.split(":", 1)[1])
        elif s.startswith("commit:"):
            commit = s.split(":", 1)[1].strip()
    if val is None:
        return None, None
    where = path.relative_to(ROOT) if path.is_relative_to(ROOT) else path
    return val, (f"{where} (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, copy-calibrated, "
                 f"at commit {commit})")


# the counter summaries of the workloads profiled on their own (bench.py --only), by (workload, tokens)
TRAFFIC = {("decode", 1): ROOT / "profiles" / "gemv_decode_b1_traffic.md",
           ("decode", 4): ROOT / "profiles" / "gemv_decode_b4_traffic.md",
           ("decode", 16): ROOT / "profiles" / "gemv_decode_b16_traffic.md",
           ("decode", 64): ROOT / "profiles" / "gemv_decode_b64_traffic.md",
           ("decode", 128): ROOT / "profiles" / "pgemm_decode_t128_traffic.md",
           ("prefill", 4096): ROOT / "profiles" / "pgemm_prefill_t4096_traffic.md",
           ("deepseek", 512): ROOT / "profiles" / "pgemm_deepseek_t512_traffic.md",
           ("skewed", 2048): ROOT / "profiles" / "pgemm_skewed_t2048_traffic.md",
           ("q4km", 4096): ROOT / "profiles" / "pgemm_q4km_t4096_traffic.md"}


def line(name: str, shape: dict, T: int, r: dict, steps: int) -> dict:
    """One workload's object: tokens/s, median / mean step, per-kernel ms, the roofline of its dominant kernel (of
    gate_up and down, the longer), the layer's."""
    w = work(shape, T, r["U"], 2 if "prefill_x" in r["names"] else 4, r["names"])
    lb, lf = w["layer"]
    mfma = lf / (MFMA_F16_PEAK_TFLOPS * 1e12) > lb / (HBM_PEAK_GBS * 1e9)  # (the layer's binding roof)
    kern = max(("gate_up", "down"), key=lambda n: r["kernels"].get(n, 0.0))
    kms = r["kernels"].get(kern, float("nan"))
    kb, kf = w[kern]
    tb, src = traffic(TRAFFIC[(name, T)], kern) if (name, T) in TRAFFIC else (None, None)
    if mfma:
        ach = kf / (kms * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": kern, "achieved": ach, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": ach / MFMA_F16_PEAK_TFLOPS, "traffic": tb, "traffic_source": src, "kernel_ms": kms,
                "algorithmic_flops": kf, "algorithmic_bytes": kb}
        la = lf / (r["ms"] * 1e-3) / 1e12
        lroof = {"bound": "mfma", "achieved": la, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": la / MFMA_F16_PEAK_TFLOPS, "algorithmic_flops": lf}
    else:
        ach = kb / (kms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": kern, "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": ach / HBM_PEAK_GBS, "traffic": tb, "traffic_source": src, "kernel_ms": kms,
                "algorithmic_bytes": kb}
        la = lb / (r["ms"] * 1e-3) / 1e9
        lroof = {"bound": "hbm", "achieved": la, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": la / HBM_PEAK_GBS,
                 "algorithmic_bytes": lb}
    names = r["names"]
    # the activations as the experts' products take them: fp16 rows (prefill tiles), int8 hi + lo planes (XQ, the
    # decode GEMV), bf16 hi + lo planes (the MFMA decode tiles)
    dtype = "f16" if "prefill_x" in names else "i8x2-xq" if any(n.startswith("router_quant") for n in names) else "bf16x2"
    return {"tokens": T, "value": T / (r["ms"] * 1e-3), "unit": "tokens/s", "ms_per_step": r["ms"],
            "ms_median_evented": r["ms_median_evented"], "steps": steps, "dtype": dtype, "experts_touched": r["U"],
            "kernel_ms": r["kernels"], "roofline": roof, "layer_roofline": lroof}


def cpu_baseline(name: str, shape: dict, T: int, threads: int | None, budget_s: float) -> dict:
    """The numpy oracle (router in float64, routing, per-expert dequantization, fp32 SwiGLU, shared expert) on the
    same workload (weight set 0, the same tokens), repeated for about ``budget_s`` seconds (at least once), BLAS
    limited to ``threads`` (None: all of the host's)."""
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import layers
    from oracle.tensors import from_bf16_bits

    spec = layers.CONFIGS[name]
    w = synth_layer(shape, 100)
    shared = (w["ffn_gate_shexp"], w["ffn_up_shexp"], w["ffn_down_shexp"]) if shape.get("shared_F") else None
    layer = layers.Layer(spec, w["ffn_gate_inp"], w["ffn_gate_exps"], w["ffn_up_exps"], w["ffn_down_exps"], shared)
    x = from_bf16_bits(synth_x(shape, T))
    times = []
    with threadpool_limits(threads):
        used = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
        t_end = time.perf_counter() + budget_s
        while not times or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            layers.forward(layer, x)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": T / med, "unit": "tokens/s", "cores": int(used), "kind": "port",
            "sample": f"{len(times)} full layer call(s) of {T} tokens (numpy oracle, {used} BLAS thread(s)), median "
                      f"{med * 1e3:.0f} ms; host {os.cpu_count()} logical CPUs"}


def commit() -> str:
    try:
        return subprocess.run(["git", "-C", str(ROOT), "rev-parse", "--short", "HEAD"], capture_output=True,
                              text=True, timeout=10).stdout.strip() or "unknown"
    except (OSError, subprocess.SubprocessError):
        return "unknown"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=16)
    ap.add_argument("--weight-sets", type=int, default=4)
    ap.add_argument("--prefill-tokens", type=int, default=4096)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the headline decode and prefill lines")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of each headline CPU baseline (0: none)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (the calibration kernel of counter profiles)")
    ap.add_argument("--only", choices=["decode", "prefill", "deepseek", "skewed", "q4km"],
                    help="run one workload alone (decode at --tokens), for profiling; prints its line object")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU (asked for {args.gpus}); the path is single-GPU by design",
              file=sys.stderr)
        sys.exit(2)

    from artlite_amd import device_count

    assert device_count() > 0, "no GPU visible"
    if args.copy_probe:
        from artlite_amd.moe.layer import hbm_copy_ms

        log(f"copy probe: {args.copy_probe} MiB, {hbm_copy_ms(args.copy_probe << 20, 1):.3f} ms")
    if args.only:
        name = args.only
        sx = SHAPES[name]
        Tx = {"decode": args.tokens, "prefill": args.prefill_tokens, "deepseek": 512, "skewed": 2048,
              "q4km": 4096}[name]
        sets = args.weight_sets if name == "decode" else 2 if name == "deepseek" else 1
        steps = args.steps if name == "decode" else args.prefill_steps
        log(f"{name}: T={Tx}, {sets} weight set(s)")
        g = build_layers(sx, sets, Tx)
        obj = line(name, sx, Tx, time_T(g, sx, Tx, steps, args.warmup), steps)
        for y in g:
            y.close()
        print(json.dumps({"workload": name, **obj}), flush=True)
        return
    shape = SHAPES["decode"]
    T = args.tokens
    batches = [T] if args.no_extra else sorted({1, 4, T, 64, 128})
    log(f"decode: T in {batches}, {args.weight_sets} weight sets")
    gls = build_layers(shape, args.weight_sets, max(batches))
    dec = {b: time_T(gls, shape, b, args.steps, args.warmup) for b in batches}
    for g in gls:
        g.close()
    head = line("decode", shape, T, dec[T], args.steps)
    out = {
        "metric": METRIC, "value": head["value"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": head["dtype"], "data": "synthetic",
        "config": {"workload": "qwen3-30b-a3b-shaped MoE layer, Q4_0 experts, decode (BASELINE config 2)",
                   "tokens": T, "hidden": shape["H"], "experts": shape["E"], "top_k": shape["k"],
                   "expert_ffn": shape["F"], "weights": shape["gate"], "activations": "bf16",
                   "weight_sets": args.weight_sets, "experts_touched": head["experts_touched"]},
        "ms_median_evented": head["ms_median_evented"], "roofline": head["roofline"],
        "layer_roofline": head["layer_roofline"],
        "kernel_ms": head["kernel_ms"], "commit": commit(),
        "decode_batches": {str(b): line("decode", shape, b, dec[b], args.steps) for b in batches if b != T},
    }
    if not args.no_prefill:
        Tp = args.prefill_tokens
        log(f"prefill: T={Tp}")
        ps = SHAPES["prefill"]
        g = build_layers(ps, 1, Tp)
        out["prefill"] = line("prefill", ps, Tp, time_T(g, ps, Tp, args.prefill_steps, args.warmup),
                              args.prefill_steps)
        g[0].close()
    extra = {}
    if not args.no_extra:
        for name, Tx, sets in (("deepseek", 512, 2), ("skewed", 2048, 1), ("q4km", 4096, 1)):
            log(f"{name}: T={Tx}")
            sx = SHAPES[name]
            g = build_layers(sx, sets, Tx)
            extra[name] = line(name, sx, Tx, time_T(g, sx, Tx, args.prefill_steps, args.warmup), args.prefill_steps)
            for y in g:
                y.close()
        out["configs"] = extra
    if args.cpu_seconds > 0:
        log("cpu baselines")
        out["cpu_baseline"] = cpu_baseline("decode", shape, T, None, args.cpu_seconds)
        out["cpu_baseline_1thread"] = cpu_baseline("decode", shape, T, 1, args.cpu_seconds)
        if "prefill" in out:
            ps = SHAPES["prefill"]
            out["prefill"]["cpu_baseline"] = cpu_baseline("prefill", ps, args.prefill_tokens, None, args.cpu_seconds)
            out["prefill"]["cpu_baseline_1thread"] = cpu_baseline("prefill", ps, args.prefill_tokens, 1, 0.0)
        short = max(2.0, args.cpu_seconds / 4)
        for b, obj in out["decode_batches"].items():
            obj["cpu_baseline"] = cpu_baseline("decode", shape, int(b), None, short)
        for name, obj in extra.items():
            obj["cpu_baseline"] = cpu_baseline(name, SHAPES[name], obj["tokens"], None, 0.0)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
