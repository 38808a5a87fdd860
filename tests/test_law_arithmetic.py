"""The float64 law arithmetic of csrc/sample.hip, checked on the CPU.

Every sampling kernel forms p(v) = exp(x_v / T - M) / S with two helpers:
LawScale (x / T as a product with 1/T plus one fused correction step) and
law_exp (a table-driven exp for z <= 0).  This test replays their exact
operation sequence in Python - fused multiply-adds are computed exactly with
Fractions and rounded once, as the hardware does - on the constants parsed
from the HIP source, and checks them against what the mathematics fixes:
  * the corrected quotient equals true IEEE division (correct rounding);
  * exp(z) is within 0.56 ulp of exp computed to 40 digits;
  * the table holds 2^(j/32) to twice double precision;
  * exp(0) = 1, exp(-inf) = exp(nan) = 0, underflow to 0 below -746.
The kernels' outputs are compared with the float64 oracle on the GPU
(tests/test_gpu_sampling.py).
"""
import math
import os
import random
import re
import struct
from decimal import Decimal, getcontext
from fractions import Fraction

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'qwen3_dspark_amd', 'csrc',
                   'sample.hip')


def _constants():
    text = open(SRC).read()
    body = re.search(r'double LAW_EXP_TAB\[64\] = \{(.*?)\};', text, re.S).group(1)
    tab = [float.fromhex(x.strip()) for x in body.replace('\n', ' ').split(',') if x.strip()]
    scalars = {name: float.fromhex(re.search(rf'constexpr double {name} = ([^;]+);', text).group(1).strip())
               for name in ('EXP_INV_L', 'EXP_L1', 'EXP_L2')}
    assert len(tab) == 64
    return tab, scalars


TAB, K = _constants()


def fma(a, b, c):
    return float(Fraction(a) * Fraction(b) + Fraction(c))


def law_div(x, T):
    """LawScale for T in [2^-100, 2^100]."""
    rT = 1.0 / T
    q = x * rT
    return fma(fma(-q, T, x), rT, q)


def law_exp(z):
    z = max(z, -746.0) if not math.isnan(z) else -746.0   # fmax: NaN yields the other operand
    k = float(round(z * K['EXP_INV_L']))                  # rint, ties to even
    n = int(k)
    r = fma(-k, K['EXP_L2'], fma(-k, K['EXP_L1'], z))
    c = fma(r, 1.0 / 720, 1.0 / 120)
    c = fma(r, c, 1.0 / 24)
    c = fma(r, c, 1.0 / 6)
    c = fma(r, c, 0.5)
    p = fma(r * r, c, r)
    hi, lo = TAB[2 * (n & 31)], TAB[2 * (n & 31) + 1]
    return math.ldexp(hi + fma(hi, p, lo), n >> 5)


def _bf16(bits):
    return struct.unpack('<f', struct.pack('<I', bits << 16))[0]


def test_table_is_two_to_the_j_over_32():
    getcontext().prec = 60
    for j in range(32):
        exact = Decimal(2) ** (Decimal(j) / 32)
        assert Decimal(TAB[2 * j]) == Decimal(float(exact))                  # hi is the rounded value
        assert abs(Decimal(TAB[2 * j]) + Decimal(TAB[2 * j + 1]) - exact) < exact * Decimal(2) ** -104


def test_reduction_constants():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    assert K['EXP_INV_L'] == float(32 / ln2)
    m, _ = math.frexp(K['EXP_L1'])
    assert (m * 2 ** 37).is_integer()                                        # k * L1 exact for |k| < 2^16
    assert abs(Decimal(K['EXP_L1']) + Decimal(K['EXP_L2']) - ln2 / 32) < Decimal(2) ** -98


def test_corrected_quotient_is_true_division():
    # every finite bf16 logit at the bench temperature
    for bits in range(1 << 16):
        x = _bf16(bits)
        if math.isfinite(x):
            assert law_div(x, 0.8) == x / 0.8, (x,)
    rng = random.Random(11)
    for _ in range(3000):
        x = struct.unpack('<f', struct.pack('<I', rng.getrandbits(32)))[0]
        if not math.isfinite(x):
            continue
        T = 2.0 ** rng.uniform(-100, 100)
        assert law_div(x, T) == x / T, (x, T)
    for T in (0.7, 1.0, 1.3, 0.3, 123.456, 2.0 ** -100, 2.0 ** 100):
        for x in (0.0, 1.0, -3.5, 65504.0, 3.4028234663852886e38, -1.401298464324817e-45):
            assert law_div(x, T) == x / T, (x, T)


def test_exp_within_056_ulp():
    getcontext().prec = 40
    rng = random.Random(3)
    worst = 0.0
    for i in range(6000):
        z = -rng.random() * (746.0, 40.0, 1.0, 1e-3)[i % 4]
        got = law_exp(z)
        ref = Decimal(z).exp()
        if ref < Decimal(2) ** -1022:
            # subnormal results: one rounding of the correctly rounded mantissa
            assert abs(Decimal(got) - ref) <= Decimal(2) ** -1074, z
            continue
        err = float(abs(Decimal(got) - ref) / Decimal(math.ulp(float(ref))))
        worst = max(worst, err)
    assert worst <= 0.56, worst


def test_exp_special_values():
    assert law_exp(0.0) == 1.0 and law_exp(-0.0) == 1.0
    assert law_exp(-746.0) == 0.0 and law_exp(-1e300) == 0.0
    assert law_exp(-math.inf) == 0.0 and law_exp(math.nan) == 0.0
    assert law_exp(-708.5) == math.exp(-708.5)                              # subnormal range
    assert law_exp(math.log(0.5)) == 0.5
