"""bench.py's contract on the CPU: the one-GPU refusal, the CPU-baseline line at
the workload's shard size, and the committed HBM-traffic figures the roofline
reads (machine-readable block against the summary's own table)."""
import json
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _run(*args, timeout=120):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_cpu_shard_line():
    r = _run("--cpu-shard", "--tokens", "384", "--head-dim", "32")
    assert r.returncode == 0, r.stderr
    line = json.loads(r.stdout.strip().splitlines()[-1])
    cpu = line["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["unit"] == "TFLOP/s"
    assert cpu["value"] > 0 and cpu["seconds"] > 0 and cpu["cores"] >= 1
    # one full hop and the diagonal: 3.5 x 4 N^2 d x 1.5
    # (value and seconds are printed rounded to 6 and 3 decimals)
    flops = 3.5 * 4.0 * 384 ** 2 * 32 * 1.5
    lo, hi = flops / (cpu["seconds"] + 5e-4) / 1e12, flops / max(cpu["seconds"] - 5e-4, 1e-9) / 1e12
    assert lo - 1e-6 <= cpu["value"] <= hi + 1e-6
    assert "384-token shards" in cpu["sample"] and "world 2 rank 1" in cpu["sample"]
    # configs 2+3 at this geometry: 7.5 hops x 16 heads of forward, 3.5x with the backward
    full = 3.5 * 4.0 * 384 ** 2 * 32 * 7.5 * 16
    assert cpu["extrapolated_full_config_s"] == pytest.approx(
        full / (cpu["value"] * 1e12), rel=2e-3, abs=0.05)


def _traffic_table():
    """(read GB, write GB, total GB) per kernel row of the committed traffic summary."""
    text = open(os.path.join(ROOT, "profiles", "hbm_traffic_ring_fwd_bwd_32k_bf16.md")).read()
    rows = {}
    for line in text.splitlines():
        m = re.match(r"\| (\w+)(?:<\d+>)? \(([a-z]+)[^|]*\| [\d,]+ \| [\d,]+ \| ([\d.]+) \| "
                     r"([\d.]+) \| ([\d.]+) \|", line)
        if m:
            rows[(m.group(1), m.group(2))] = tuple(float(m.group(i)) for i in (3, 4, 5))
    return rows


def test_committed_traffic_matches_its_table():
    rows = _traffic_table()
    pair = bench.measured_traffic("dkdv128_kernel + dqds128_kernel (dS shared)", 32768, 16, 128)
    dkdv, dqds = rows[("dkdv128_kernel", "full")], rows[("dqds128_kernel", "full")]
    assert pair == pytest.approx((dkdv[2] + dqds[2]) * 1e9, rel=1e-3)
    fwd = bench.measured_traffic("fwd128_kernel", 32768, 16, 128)
    assert fwd == pytest.approx(rows[("fwd128_kernel", "full")][2] * 1e9, rel=1e-3)
    # read + write = total in every row the block draws on
    for r in (dkdv, dqds):
        assert r[0] + r[1] == pytest.approx(r[2], abs=2e-3)
    # no committed figure for other shapes
    assert bench.measured_traffic("dkdv128_kernel + dqds128_kernel", 1024, 16, 128) is None


def test_algorithmic_floor_of_the_pair():
    n, h, d = 32768, 16, 128
    floor = bench.algorithmic_bytes("dkdv128_kernel + dqds128_kernel", n, h, d)
    # bf16 Q, dO, K, V; fp32 LSE and delta; fp32 dQ, dK, dV read and written
    assert floor == 4 * n * h * d * 2 + 2 * n * h * 4 + 6 * n * h * d * 4
    assert floor / 1e9 == pytest.approx(2.152, abs=1e-3)
    fwd = bench.algorithmic_bytes("fwd128_kernel<8>", n, h, d)
    assert fwd / 1e9 == pytest.approx(0.947, abs=1e-3)
    assert bench.algorithmic_bytes("merge_rows_kernel", n, h, d) == 0
