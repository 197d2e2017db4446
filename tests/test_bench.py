"""bench.py's host side (CPU): the ops convention, the prologue's algorithmic bytes, the committed
traffic figure it reports, the metric name, and the one-GPU refusal. The timed run itself needs a
GPU and is the driver's."""
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_metric_is_baselines(bench):
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        assert bench.METRIC == json.load(f)["metric"]


def test_ops_convention(bench):
    # 4*B*H*N^2*D, halved when causal (the reference's bench/bench_attention.py:140): the figures
    # the targets are quoted on
    assert bench.ops_of(1, 48, 47520, True) == pytest.approx(2.7748e13, rel=1e-4)
    assert bench.ops_of(1, 48, 47520, False) == pytest.approx(5.5496e13, rel=1e-4)
    assert bench.ops_of(1, 48, 8771, False) == pytest.approx(1.89e12, rel=2e-3)
    assert bench.ops_of(1, 48, 16384, True) == pytest.approx(3.30e12, rel=2e-3)
    assert bench.ops_of(8, 24, 4096, False) == pytest.approx(1.65e12, rel=2e-3)
    assert bench.ops_of(1, 10, 4096, False, D=64) == 4.0 * 10 * 4096 * 4096 * 64


def test_prologue_bytes_headline(bench):
    # K read twice (mean, quant) + V once, fp16; K8 + V8T written (N_pad = 47552); SK and SV
    # written, SV read and rewritten by the fold (4 fp32 passes over B*H*N_pad)
    el = 48 * 47520 * 128 * 2
    q8 = 48 * 47552 * 128
    assert bench.prologue_bytes(1, 48, 47520) == 3 * el + 2 * q8 + 4 * 48 * 47552 * 4 == 2372616192
    assert bench.prologue_bytes(1, 48, 47520, smooth_k=False) == 2372616192 - el


def test_profiled_traffic_is_the_committed_figure(bench):
    t = bench.profiled_traffic("c3c")
    assert isinstance(t, int)
    # at least the main loop's algorithmic bytes (Q, K8, V8T, KCONST read; O written) ...
    algorithmic = 48 * 47520 * 128 * 2 * 2 + 2 * 48 * 47552 * 128 + 48 * 47552 * 3 * 4
    assert algorithmic <= t <= 3 * algorithmic
    # ... and exactly the number the profile states
    with open(os.path.join(ROOT, "profiles", "attn_fwd_c3c_hbm_traffic.md")) as f:
        assert ("traffic_bytes_per_launch[c3c] = %d" % t) in f.read()
    assert bench.profiled_traffic("c1") is None


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""
