"""bench.py's side of the measurement contract that needs no GPU: the metric
it reports is BASELINE.json's, the peaks it divides by are MI355X's
published dense figures, and a request for more than one GPU is refused
with a message (this build runs on one GPU).  The bench itself runs on the
MI355X box.
"""
from __future__ import annotations

import json
import subprocess
import sys

import bench
from conftest import ROOT


def test_metric_is_the_baselines():
    want = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    assert bench.METRIC == want


def test_peaks_are_mi355x_dense_figures():
    assert bench.PEAK_BF16_TFLOPS == 2516.6  # 256 CUs x 2.4 GHz x 4096 bf16 flop/clk/CU
    assert bench.PEAK_HBM_GBS == 8000.0
    assert bench.PEAK_INT8_TOPS == 5000.0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]
