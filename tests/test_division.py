"""The prologue's per-element quotient RN(x / s) is computed as

    y = RN(1 / s)            (one correctly rounded division per row, or a constant)
    q = RN(x * y)
    e = RN(q * s - x)        (fma: exact)
    r = RN(q - e * y)        (fma)

(`div_by` in csrc/sage_device.h), which must equal the correctly rounded division the reference's
quantizers use (kernels/hip/h34_prologue.hip:147-157, :186-196; built without fast-math,
tools/build_hsaco.py:118-120) bit for bit, on the inputs the quantizers give it: a row value over
the row's scale (|x / s| <= 127 or 448 up to rounding) and the row absmax over 127 or 448.

These CPU tests emulate the four fp32 operations exactly (products of two fp32 values are exact in
fp64; the final sum is rounded once with an exact two-sum and a midpoint check) and compare with
numpy's IEEE fp32 division on random, near-tie and boundary inputs. The GPU parity tests then hold
the kernels' quantized tensors bit-exact against the oracle.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

f32, f64 = np.float32, np.float64


def _rn32_of_sum(a, b):
    """RN32(a + b) of float64 a and b, exactly."""
    s = a + b
    bb = s - a
    err = (a - (s - bb)) + (b - bb)          # s + err == a + b exactly (two-sum)
    r = s.astype(f32)
    r64 = r.astype(f64)
    up = np.nextafter(r, np.inf, dtype=f32)
    dn = np.nextafter(r, -np.inf, dtype=f32)
    at_up = s == (r64 + up.astype(f64)) / 2   # s is the midpoint above r: err decides
    at_dn = s == (r64 + dn.astype(f64)) / 2
    out = r.copy()
    m = at_up & (err > 0)
    out[m] = up[m]
    m = at_dn & (err < 0)
    out[m] = dn[m]
    return out


def div_by(x, s, y):
    """The device sequence, with every fp32 operation rounded once."""
    q = (x * y).astype(f32)
    e = (q.astype(f64) * s.astype(f64) - x.astype(f64)).astype(f32)   # exact in fp64, one rounding
    return _rn32_of_sum(q.astype(f64), -(e.astype(f64) * y.astype(f64)))


def _check(x, s):
    y = (f32(1) / s).astype(f32)
    got = div_by(x, s, y)
    ref = (x / s).astype(f32)
    bad = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, list(zip(x[bad[:5]], s[bad[:5]], ref[bad[:5]], got[bad[:5]]))


@pytest.mark.parametrize("top", [127.0, 448.0])
def test_row_quotients_random(top):
    rng = np.random.default_rng(11 if top == 127.0 else 12)
    n = 1_000_000
    kmax = np.exp(rng.uniform(np.log(1e-9), np.log(5e4), n)).astype(f32)
    x = (rng.uniform(-1, 1, n) * kmax).astype(f32)
    x[: n // 10] = kmax[: n // 10]                       # the row's own absmax: quotient ~ top
    x[n // 10: n // 5] = -kmax[n // 10: n // 5]
    s = np.maximum((kmax / f32(top)).astype(f32), f32(1e-12))
    _check(x, s)


def test_row_quotients_near_ties():
    """Quotients within a few ulps of k + 1/2: where a wrong last bit changes the int8 byte."""
    rng = np.random.default_rng(13)
    n = 1_000_000
    s = np.exp(rng.uniform(np.log(1e-6), np.log(10), n)).astype(f32)
    k = rng.integers(-128, 128, n)
    x = ((k + 0.5) * s.astype(f64)).astype(f32)
    x = (x.view(np.int32) + rng.integers(-4, 5, n).astype(np.int32)).view(f32)
    _check(x, s)


def test_floor_scale_rows():
    """Rows whose scale is the 1e-12 floor: tiny values over the floor."""
    rng = np.random.default_rng(14)
    n = 200_000
    x = (rng.uniform(-1, 1, n) * 1.2e-10).astype(f32)
    _check(x, np.full(n, 1e-12, f32))


@pytest.mark.parametrize("top", [127.0, 448.0])
def test_constant_divisor_windows(top):
    """Scale computation RN(absmax / top): every fp32 bit pattern in random windows."""
    rng = np.random.default_rng(15)
    for base in rng.integers(0x00800000, 0x7E000000, 4):
        x = (np.arange(250_000, dtype=np.int64) + int(base)).astype(np.int32).view(f32)
        _check(x, np.full(x.shape, top, f32))


def test_signed_zero():
    s = np.array([0.5, 3.0, 1e-12], f32)
    for z in (0.0, -0.0):
        got = div_by(np.full(3, z, f32), s, (f32(1) / s).astype(f32))
        assert (got == 0).all() and (np.signbit(got) == np.signbit(f32(z))).all()


def test_emulation_detects_a_one_ulp_slip():
    """The checker itself: a quotient one ulp off must be reported."""
    x = np.array([3.0], f32)
    s = np.array([7.0], f32)
    ref = (x / s).astype(f32)
    assert np.nextafter(ref, np.inf, dtype=f32).view(np.uint32) != ref.view(np.uint32)
    y = (f32(1) / s).astype(f32)
    assert div_by(x, s, y).view(np.uint32)[0] == ref.view(np.uint32)[0]
    # dropping the correction step (q alone) is wrong somewhere in a modest sample
    rng = np.random.default_rng(16)
    xs = rng.uniform(-100, 100, 100_000).astype(f32)
    ss = rng.uniform(0.01, 2, 100_000).astype(f32)
    q = (xs * (f32(1) / ss).astype(f32)).astype(f32)
    assert (q != (xs / ss).astype(f32)).any()


@pytest.fixture(scope="module")
def div_exhaustive(tmp_path_factory):
    """tests/native/div_exhaustive.c built with gcc (OpenMP over the host's cores)."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "div_exhaustive.c")
    exe = str(tmp_path_factory.mktemp("divx") / "div_exhaustive")
    subprocess.run([gcc, "-O2", "-fopenmp", "-o", exe, src, "-lm"], check=True)

    def run(*args):
        out = subprocess.run([exe] + [str(a) for a in args], check=True, capture_output=True,
                             text=True, timeout=600).stdout
        words = out.split("\n")[0].split()
        return dict(zip(words[0::2], words[1::2])), out
    return run


def test_constant_divisor_127_exhaustive(div_exhaustive):
    # every non-negative finite fp32 x (2^31 - 2^23 inputs): RN(x/127) bit for bit, subnormal
    # quotients included -- the int8 scale max(RN(kmax/127), 1e-12)
    r, out = div_exhaustive(127, 1e-12)
    assert int(r["checked"]) == 0x7f800000
    assert int(r["mismatches"]) == 0, out


def test_constant_divisor_448_exhaustive(div_exhaustive):
    # every non-negative finite fp32 x: RN(x/448) bit for bit wherever the quotient is a normal
    # number; where it is subnormal (x < 448 * 2^-126) the correction step is not exact, but
    # those quotients lie far below the scales' 1e-12 floor, so max(RN(x/448), 1e-12) -- the
    # e4m3 scales sv and sk -- is exact for every x
    r, out = div_exhaustive(448, 1e-12)
    assert int(r["checked"]) == 0x7f800000
    assert int(r["normal_quotient_mismatches"]) == 0, out
    assert int(r["floored_mismatches"]) == 0, out
    assert float.fromhex(r["max_bad_x"]) < 448 * 2.0 ** -126


@pytest.mark.parametrize("variant", [1, 2], ids=["no_correction", "unfused_residual"])
def test_exhaustive_check_catches_a_planted_mistake(div_exhaustive, variant):
    # the plausible shortcuts -- q = RN(x * RN(1/s)) alone, or a residual formed with two
    # roundings -- must show normal-range mismatches for both divisors (a reciprocal a few ulps
    # off RN(1/s) does not: the exact-residual correction absorbs it)
    for top in (127, 448):
        r, out = div_exhaustive(top, 1e-12, variant)
        assert int(r["normal_quotient_mismatches"]) > 0, out
