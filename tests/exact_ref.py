"""Independent exact-arithmetic restatements used to pin the oracle (CPU only).

Nothing here calls torch arithmetic: values are Python `Fraction`s and results are rounded by
explicit rules, so a check of the oracle against these functions tests the oracle's torch ops
(division vs reciprocal, rounding rules, operation order) and not a retyping of them.

* `rn32(x)`   -- IEEE binary32 round-to-nearest-even of an exact rational (normals and subnormals);
* `e4m3_code(x)` -- the OCP 8-bit float E4M3FN encoding (bias 7, 3 mantissa bits, max 448, no
  infinities, S.1111.111 = NaN), round-to-nearest-even, from the OCP FP8 specification;
* `rne_int(x)` -- round half to even to an integer.
"""
import bisect
import math
import struct
from fractions import Fraction


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def rn32(x) -> float:
    """Round an exact rational to the nearest binary32 value, ties to even."""
    x = Fraction(x)
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)                         # subnormal range: fixed quantum 2^-149
    quantum = Fraction(2) ** (e - 23)
    m = a / quantum
    r = round(m)                             # Fraction.__round__: half to even
    val = r * quantum
    if val >= Fraction(2) ** 128:
        return sign * math.inf
    return sign * float(val)


def rne_int(x) -> int:
    return round(Fraction(x))


def _e4m3_values():
    vals = []
    for code in range(0x7F):                  # 0x7F is NaN
        e, m = code >> 3, code & 7
        if e == 0:
            v = Fraction(m, 8) * Fraction(2) ** -6
        else:
            v = (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
        vals.append((v, code))
    return vals


_E4M3 = _e4m3_values()


_E4M3_VALS = [v for v, _ in _E4M3]


def e4m3_code(x) -> int:
    """OCP E4M3FN byte of `x`, round to nearest even; |x| must be <= 448 (plus its half-ulp).

    A float -0.0 encodes as 0x80 (negative zero), like any negative value that rounds to zero."""
    neg = (x < 0) or (isinstance(x, float) and x == 0 and math.copysign(1.0, x) < 0)
    x = Fraction(x)
    sign = 0x80 if neg else 0
    a = abs(x)
    if a > 464:
        raise ValueError("out of the range this encoder serves")
    i = bisect.bisect_left(_E4M3_VALS, a)
    cands = [j for j in (i - 1, i) if 0 <= j < len(_E4M3_VALS)]
    best = None
    for j in cands:
        v, code = _E4M3[j]
        d = abs(a - v)
        if best is None or d < best[0] or (d == best[0] and (code & 1) == 0):
            best = (d, code)
    return sign | best[1]


def e4m3_value(code: int) -> Fraction:
    s = -1 if code & 0x80 else 1
    return s * dict((c, v) for v, c in _E4M3)[code & 0x7F]
