"""Host logic of bench.py (no GPU): the roofline object of a measurement,
the operand type it reports, the expert byte counts, and the refusal of a
multi-GPU run."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from tie_amd import synth  # noqa: E402


def measurement(ms, kernels):
    return {"ms": ms, "kernels": kernels}


def test_expert_bytes_of_the_30b_shape():
    cfg = synth.CONFIGS["30b_t32"]
    gu, dn = bench.expert_bytes(cfg)
    # Q4_K: 144 bytes per 256 weights; Q6_K: 210 bytes per 256 weights
    assert gu == 2 * 768 * (2048 // 256) * 144
    assert dn == 2048 * (768 // 256) * 210


def test_roofline_picks_the_longest_kernel_and_its_bound():
    # an HBM-bound kernel: 198 MB in 50 us = 3960 GB/s
    hbm = {"avg_us": 50.0, "alg_bytes": 198e6, "GBps": 3960.0, "alg_flops": 3.2e9, "TFLOPs": 64.0}
    short = {"avg_us": 10.0, "alg_bytes": 4e6, "GBps": 400.0, "alg_flops": None, "TFLOPs": None}
    fix = {"avg_us": 99.0, "alg_bytes": None, "GBps": None, "alg_flops": None, "TFLOPs": None}
    r = bench.roofline(measurement(0.11, {"mfma_gate_up": hbm, "router": short, "recompute": fix}), "nope")
    # the kernel without an algorithmic byte count is no candidate
    assert r["kernel"] == "mfma_gate_up"
    # intensity 3.2e9 / 198e6 = 16 flop/B, below the ridge (2.5e15 / 8e12 = 312.5): HBM
    assert r["bound"] == "hbm" and r["unit"] == "GB/s"
    assert r["frac"] == pytest.approx(3960.0 / 8000.0, abs=1e-4)
    assert r["kernel_le_step"] is True
    assert r["traffic"] is None  # no such workload in profiles/traffic.json


def test_roofline_mfma_bound_and_kernel_longer_than_step():
    k = {"avg_us": 140.0, "alg_bytes": 2.6e8, "GBps": 1857.0, "alg_flops": 1.03e11, "TFLOPs": 736.0}
    r = bench.roofline(measurement(0.12, {"mfma_gate_up": k}), "nope")
    # 1.03e11 / 2.6e8 = 396 flop/B, above the ridge: the matrix-core bound
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
    assert r["frac"] == pytest.approx(736.0 / 2500.0, abs=1e-4)
    # a 140 us kernel cannot fit a 0.12 ms step: the cross-check says so
    assert r["kernel_le_step"] is False


def test_compute_dtype():
    assert bench.compute_dtype({"kernels": {"mfma_gate_up": {}}}, synth.CONFIGS["30b_t32"]) == "f16"
    assert bench.compute_dtype({"kernels": {"mfma_gate_up": {}}}, synth.CONFIGS["30b_bf16_zipf_t512"]) == "bf16"
    assert bench.compute_dtype({"kernels": {"exact_gate_up": {}}}, synth.CONFIGS["30b_t8"]) == "f32"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
