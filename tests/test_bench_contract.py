"""bench.py's contract on the CPU: one GPU only (N > 1 exits with a message,
before any device work), and the byte accounting behind the roofline object.
The byte counts are checked against the 4-bit affine format's arithmetic
(packed nibbles, one bf16 scale and bias per 64 weights), not retyped."""

import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU only" in res.stderr
    assert res.stdout.strip() == ""   # no JSON line for a refused run


def test_qmv_bytes_cfg1():
    # x [4, 5120] . W [17408, 5120]: 17408*5120 nibbles, 17408*80 groups of
    # (scale, bias) bf16, x and y in bf16.
    M, N, K = 4, 17408, 5120
    weights = N * K // 2
    groups = N * (K // 64)
    assert bench._qmv_bytes(M, N, K, 64) == weights + groups * 4 + M * K * 2 + M * N * 2 == 50_315_264


def test_gate_up_bytes_cfg3():
    # Two matrices of the cfg1 shape, one x, the RMSNorm weight, one y.
    M, N, K = 4, 17408, 5120
    one = bench._qmv_bytes(M, N, K, 64) - M * K * 2 - M * N * 2
    assert bench._gate_up_bytes(M, N, K, 64) == 2 * one + M * K * 2 + K * 2 + M * N * 2 == 100_460_544


def test_committed_traffic_is_read():
    t = bench.measured_traffic()
    assert t is not None
    alg = bench._gate_up_bytes(4, 17408, 5120, 64)
    assert alg <= t < 1.2 * alg   # counters read at least the algorithmic bytes, and no large re-read
