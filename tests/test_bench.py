"""The benchmark's host side, on the CPU: its single-GPU contract, and that every workload it reports a roofline for
finds its kernels' HBM traffic in the counter summaries under profiles/ (the line's ``roofline.traffic``)."""

import subprocess
import sys

import pytest

import bench


def test_more_than_one_gpu_exits_with_a_message() -> None:
    r = subprocess.run([sys.executable, str(bench.ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


@pytest.mark.parametrize("key", sorted(bench.TRAFFIC))
def test_traffic_summaries_cover_both_products(key: tuple) -> None:
    path = bench.TRAFFIC[key]
    assert path.is_file(), path
    for kernel in ("gate_up", "down"):
        val, src = bench.traffic(path, kernel)
        assert val is not None and val > 0, (key, kernel)
        assert "commit" in src


def test_traffic_reads_the_summary_line(tmp_path) -> None:
    p = tmp_path / "t.md"
    p.write_text("# x\n\ncommit: abc1234\n\n- traffic_bytes_per_launch[gate_up]: 123456\n")
    val, src = bench.traffic(p, "gate_up")
    assert val == 123456.0 and "abc1234" in src
    assert bench.traffic(p, "down") == (None, None)
    assert bench.traffic(tmp_path / "missing.md", "gate_up") == (None, None)


def test_work_counts_each_product_once() -> None:
    """The layer's algorithmic bytes are its products' plus the router's weights, x in and y out; the flops of the
    two products add up to the layer's expert flops."""
    shape = bench.SHAPES["decode"]
    H, E, F, k, T, U = shape["H"], shape["E"], shape["F"], shape["k"], 16, 80.0
    names = ["router_quant", "gate_up", "down", "combine"]
    w = bench.work(shape, T, U, 4, names)
    (gb, gf), (db, df), (lb, lf) = w["gate_up"], w["down"], w["layer"]
    assert lb == pytest.approx(gb + db + E * H * 4 + T * H * 4)
    assert gf + df == pytest.approx(2.0 * T * k * 3 * H * F)
    assert lf == pytest.approx(gf + df + 2.0 * T * H * E)
