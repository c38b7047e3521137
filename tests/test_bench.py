"""bench.py on the CPU: the one-GPU refusal, the algorithmic work figures the
roofline divides by, and the CPU-baseline record (nothing here touches a GPU).

The work figures are closed forms of the configurations: 17 products of
2*8192*4096*4096 FLOP for config 5 (6 forward, 6 dW, 5 dX: the input needs no
gradient), 3.351 GFLOP for config 4 and 12.85 MFLOP for config 1 (forward and
dW only), 24 bytes per element for the config-2 chain (its fused floor) and
28 per parameter for Adam (read p, g, m, v; write p, m, v).
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_gemm_flops_per_step_are_the_closed_forms():
    batch, widths, init = bench.CONFIGS["c5"]
    assert bench.step_flops(batch, widths, init == "readme") == 17 * 2.0 * 8192 * 4096 * 4096
    batch, widths, init = bench.CONFIGS["c4"]
    c4 = 2.0 * 1024 * 784 * 1024 * 2 + 2.0 * 1024 * 1024 * 10 * 3
    assert bench.step_flops(batch, widths, init == "readme") == c4
    assert abs(c4 - 3.351e9) < 1e6
    batch, widths, init = bench.CONFIGS["c1"]
    assert bench.step_flops(batch, widths, init == "readme") == 2 * 2.0 * 32 * 784 * 128  # 12.85 MFLOP


def test_bandwidth_work_per_unit():
    # config 2's fused floor: a, b, c read once, ga, gb, gc written once (the
    # reference's op-by-op sequence moves 148: forward add/mul/div/sub 12 B each,
    # relu 8, sum 4; backward fill 4, relu mask 12, neg 8, div 20, mul 20, two
    # accumulations 12 + 12)
    assert bench.CHAIN_BYTES_PER_ELEM == 3 * 4 + 3 * 4
    assert bench.ADAM_BYTES_PER_PARAM == 4 * 4 + 3 * 4


@pytest.mark.parametrize("cfg", ["c1", "c4"])
def test_cpu_baseline_record(cfg):
    r = bench.cpu_baseline(cfg, 64)
    assert r["kind"] == "port" and r["cores"] == 1 and r["unit"] == "steps/s"
    assert r["value"] > 0
    assert set(r["breakdown_s"]) == {"gemm_s", "elementwise_s", "adam_s"}
    assert abs(1.0 / r["value"] - sum(r["breakdown_s"].values())) < 1e-3 + 0.01 / r["value"]
    host = r["host"]
    assert host["host_cores"] >= host["usable_cores"] >= 1 and host["cpu_model"]


def test_traffic_from_the_committed_counters():
    # config 3: one Adam launch per step reads and writes each operand once, so
    # the counted HBM bytes match 28 B per parameter of 2^28 parameters
    traffic, src = bench.pmc_traffic("c3")
    assert src == "profiles/c3_adam_pmc.md"
    assert abs(traffic / (28 * 2 ** 28) - 1.0) < 0.01
    traffic, src = bench.pmc_traffic("c5")
    assert src == "profiles/c5_gemm_pmc.md" and traffic > 0
    # config 2: the one compiled pass per step moves the fused floor, 24 B
    # per element of 2^26
    traffic, src = bench.pmc_traffic("c2")
    assert src == "profiles/c2_map_pmc.md"
    assert abs(traffic / (24 * 2 ** 26) - 1.0) < 0.01


def test_a_default_run_covers_every_baseline_config():
    # config 5 is the headline; the others are measured in the same run with
    # their own step counts (config 3 at the full 2^28 parameters)
    names = [c for c, _, _ in bench.OTHER_CONFIGS]
    assert sorted(names + ["c5"]) == ["c1", "c2", "c3", "c4", "c5"]
    assert all(steps > 0 and warmup >= 0 for _, steps, warmup in bench.OTHER_CONFIGS)
    assert bench.ADAM_P == 1 << 28 and bench.CHAIN_N == 1 << 26
