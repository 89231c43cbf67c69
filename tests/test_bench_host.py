"""CPU-only checks of bench.py's contract: it refuses more than one GPU, its CPU baseline (the oracle over a
workload's rows on this host) runs and reports the host it ran on, and its rates are the algorithmic work
over the measured time."""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from minillm import workloads  # noqa: E402


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_refuses_more_than_one_gpu(gpus):
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", gpus], capture_output=True, text=True,
                         timeout=120, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout.strip() == ""  # no JSON line for a configuration it does not measure


def test_cpu_baseline_on_the_smallest_workload():
    wl = workloads.decode_4()
    t, times = bench.cpu_step_seconds(wl, threads=2, reps=2)
    assert len(times) == 2 and all(x > 0 for x in times)
    assert min(times) <= t <= max(times)
    args = type("A", (), {"cpu_threads": 2})()
    line = bench.cpu_baseline(wl, args)
    assert line["kind"] == "port" and line["cores"] == 2 and line["unit"] == "tokens/s"
    assert line["value"] > 0 and line["os_cpu_count"] == os.cpu_count()
    assert isinstance(line["cpu_model"], str) and line["cpu_model"]
    assert f"all {len(wl.seqs)} rows" in line["sample"]


def test_kernel_rates_are_algorithmic_work_over_time():
    class Work:  # a workload's measured quantities, as kernel_rates reads them
        num_tokens, seqs = 4476, [None] * 128

        def decode_kernel_bytes(self, kv_elem):
            return 2_137_093_012 * kv_elem // 2

        def prefill_flops(self):
            return 51_378_782_208

    wl = Work()
    r = {"step_ms": 0.5, "dec_ms": 0.4, "pf_ms": 0.1, "forward_ms": 0.52}
    out = bench.kernel_rates(wl, r, 2)
    assert out["decode_gbps"] == pytest.approx(2_137_093_012 / 0.4e-3 / 1e9, rel=1e-3)
    assert out["decode_frac_of_8tbps"] == pytest.approx(out["decode_gbps"] / bench.HBM_PEAK_GBPS, rel=1e-3)
    assert out["prefill_tflops"] == pytest.approx(51_378_782_208 / 0.1e-3 / 1e12, rel=1e-3)
    assert out["prefill_frac_of_bf16_peak"] == pytest.approx(out["prefill_tflops"] / bench.BF16_PEAK_TFLOPS, rel=1e-3)
    assert out["step_us"] == pytest.approx(500.0) and out["forward_us"] == pytest.approx(520.0)
    assert out["tokens"] == 4476 and out["rows"] == 128
