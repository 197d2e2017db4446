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
    algorithmic = 48 * 47520 * 128 * 2 * 2 + 2 * 48 * 47552 * 128 + 48 * 47552 * 2 * 4
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


class _FakeClock:
    """A fake host clock that advances by `dt` seconds per call made, and a shader clock that
    rises by `step` MHz per reading until `top`."""

    def __init__(self, dt, mhz0=1800, step=100, top=2200):
        self.t, self.dt, self.calls = 0.0, dt, 0
        self.mhz, self.step, self.top = mhz0, step, top

    def call(self):
        self.calls += 1
        self.t += self.dt

    def now(self):
        return self.t

    def sclk(self):
        m = self.mhz
        self.mhz = min(self.top, self.mhz + self.step)
        return m


def test_settle_floor_is_time_and_calls(bench):
    # fast calls: the 4 s floor, not the call count, ends the floor phase
    fc = _FakeClock(dt=0.001, step=0)
    st = bench.settle(fc.call, lambda: None, min_calls=40, min_s=4.0, max_s=10.0,
                      clock=fc.sclk, now=fc.now)
    assert st["seconds"] >= 4.0 and st["calls"] >= 4000
    # the clock stopped rising at once: one half-second chunk after the floor, then stop
    assert st["seconds"] < 4.6
    # slow calls: the 40-call floor, not the time, ends it
    fc = _FakeClock(dt=0.5, step=0)
    st = bench.settle(fc.call, lambda: None, min_calls=40, min_s=4.0, max_s=10.0,
                      clock=fc.sclk, now=fc.now)
    assert st["calls"] >= 40 and st["seconds"] >= 20.0


def test_settle_continues_while_the_clock_rises(bench):
    fc = _FakeClock(dt=0.01, mhz0=1800, step=50, top=2100)
    st = bench.settle(fc.call, lambda: None, min_calls=40, min_s=2.0, max_s=10.0,
                      clock=fc.sclk, now=fc.now)
    # readings 1800 (start), 1850 (after the floor), then one per chunk while rising: 1900 ..
    # 2100 (5 chunks), then 2100 again (not above, a 6th chunk) ends it
    assert st["sclk_mhz"] == [1800, 1850, 1900, 1950, 2000, 2050, 2100, 2100]
    assert 2.0 + 6 * 0.5 <= st["seconds"] <= 2.0 + 6 * 0.5 + 7 * 0.01  # one call over per phase
    # bounded by max_s and by max_calls however the clock behaves
    fc = _FakeClock(dt=0.01, step=10, top=10 ** 9)
    st = bench.settle(fc.call, lambda: None, min_calls=40, min_s=2.0, max_s=3.0,
                      clock=fc.sclk, now=fc.now)
    assert st["seconds"] <= 3.0 + 0.5 + 0.02
    fc = _FakeClock(dt=0.0, step=0)
    st = bench.settle(fc.call, lambda: None, min_calls=40, min_s=2.0, max_s=3.0,
                      clock=fc.sclk, now=fc.now, max_calls=500)
    assert st["calls"] == 500
    # an unreadable clock: the floor only, plus one chunk
    fc = _FakeClock(dt=0.01)
    st = bench.settle(fc.call, lambda: None, min_s=2.0, clock=lambda: None, now=fc.now)
    assert st["sclk_mhz"][0] is None and st["seconds"] <= 2.0 + 0.5 + 0.02


class _FakeEvent:
    """Events on a fake device clock: each call takes `cost(i)` ms, recorded when it is made."""
    device_ms = 0.0

    def record(self):
        self.t = _FakeEvent.device_ms

    def elapsed_time(self, other):
        return other.t - self.t


def test_aa_twin_interleaves_and_reports_medians(bench):
    order = []
    state = {"n": 0}

    def call():
        # a clock ramp: every call 1 % cheaper than the one before
        _FakeEvent.device_ms += 10.0 * (0.99 ** state["n"])
        state["n"] += 1
        order.append(state["n"])

    _FakeEvent.device_ms = 0.0
    aa = bench.aa_twin(call, _FakeEvent, lambda: None, rounds=10, batch=3)
    assert aa["rounds"] == 10 and aa["batch"] == 3 and state["n"] == 60
    # interleaving with the order swapped each round keeps the ratio near 1 under the ramp
    # (a sequential A-then-B would report B ~25 % faster)
    assert abs(aa["ratio"] - 1.0) < 0.05
    assert 5.0 < aa["ms_a"] < 10.0 and 5.0 < aa["ms_b"] < 10.0
    for k in ("range_a", "range_b"):
        lo, hi = aa[k]
        assert lo <= hi and lo <= aa["ms_" + k[-1]] <= hi


def test_board_power_reads_hwmon(bench, tmp_path):
    # power1_average in microwatts, else power1_input; the cap beside it; the first card with a
    # power reading wins
    h0 = tmp_path / "card0" / "device" / "hwmon" / "hwmon2"
    h0.mkdir(parents=True)
    (h0 / "temp1_input").write_text("50000\n")
    h1 = tmp_path / "card1" / "device" / "hwmon" / "hwmon5"
    h1.mkdir(parents=True)
    (h1 / "power1_input").write_text("1331500000\n")
    (h1 / "power1_cap").write_text("1400000000\n")
    assert bench.board_power(str(tmp_path)) == {"watts": 1331.5, "cap_watts": 1400.0}
    (h1 / "power1_average").write_text("1200000000\n")
    assert bench.board_power(str(tmp_path))["watts"] == 1200.0
    assert bench.board_power(str(tmp_path / "nothing")) is None


def test_first_call_latency_reports_a_child_failure(bench):
    # The first-call figure comes from a fresh child process; where it cannot run (no GPU here)
    # the field carries the reason instead of a number, and the parent goes on.
    out = bench.first_call_latency("c1", timeout_s=300)
    if "error" in out:
        assert "child exited" in out["error"] or "timed out" in out["error"]
    else:
        assert out["first_call_s"] > 0 and out["library_load_s"] >= 0
