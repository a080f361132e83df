"""The per-channel quantiser's division-free quotient (CPU only).

The per-channel encoder (chan_encode_w in pitch_channel.hip) needs t = RN(RN((x - lo) / step) + 0.5) in float32
(reference/pitch_reference.py:157) and the step RN((hi - lo) / (2^b - 1)) (pitch_reference.py:155). It forms
both without dividing per element:

    step:      s0 = RN(d * RN(1 / L)),  s = RN(s0 + RN-exact(d - s0 * L) * RN(1 / L))       (two fmas)
    quotient:  q0 = RN(a * inv),        q  = RN(q0 + RN-exact(a - q0 * step') * inv)     (two fmas)

with inv = RN(1 / step) from one correctly rounded division per channel and step' = min(step, FLT_MAX).
Markstein's theorem makes q the correctly rounded quotient. These tests restate that arithmetic with an exact
fma (rational arithmetic rounded once to float32, ties to even) and check it against numpy's correctly rounded
float32 division, on the operand ranges the codec sees: fp16-rounded ranges, steps for 2..8 bits, values inside
the range, at its ends and constructed next to every rounding point of t. A plausible slip (a missing
correction term, the wrong operand in the residual, an uncorrected product) fails them.
"""
from fractions import Fraction

import numpy as np
import pytest

f32 = np.float32
FLT_MAX = np.finfo(np.float32).max


def rn32(x: Fraction) -> float:
    """x rounded to the nearest float32 (ties to even), as a Python float; x finite and in range."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    e = max(e, -126)                       # subnormals share the smallest exponent
    m = x * Fraction(2) ** (23 - e)        # 24-bit significand scale
    q, r = divmod(m.numerator, m.denominator)
    if 2 * r > m.denominator or (2 * r == m.denominator and q % 2 == 1):
        q += 1
    return sign * float(Fraction(q) * Fraction(2) ** (e - 23))


def fma32(a, b, c) -> float:
    return rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_rn32_matches_numpy():
    rng = np.random.default_rng(0)
    for v in rng.standard_normal(2000) * np.exp(rng.uniform(-30, 30, 2000)):
        assert rn32(Fraction(float(v))) == float(f32(v))
    # ties: 1 + 2^-24 lies halfway between 1 and 1 + 2^-23 and rounds to even (1)
    assert rn32(Fraction(1) + Fraction(1, 2 ** 24)) == 1.0
    assert rn32(Fraction(1) + Fraction(3, 2 ** 24)) == float(f32(1) + f32(2 ** -22))


def kivi_step(d: float, bits: int) -> float:
    L = float(2 ** bits - 1)
    il = float(f32(1) / f32(L))
    s0 = float(f32(d) * f32(il))
    s = fma32(fma32(-s0, L, d), il, s0)
    return 1.0 if s == 0.0 else s


def quotient(a: float, step: float) -> float:
    inv = float(f32(1) / f32(step))
    q0 = float(f32(a) * f32(inv))
    return fma32(fma32(-q0, min(step, float(FLT_MAX)), a), inv, q0)


def ranges(bits, n, seed):
    rng = np.random.default_rng(seed)
    lo = rng.standard_normal(n) * np.exp(rng.uniform(-8, 10, n))
    width = np.exp(rng.uniform(-12, 10, n))
    lo16 = np.clip(lo, -65504, 65504).astype(np.float16).astype(f32)
    hi16 = np.clip(lo + width, -65504, 65504).astype(np.float16).astype(f32)
    return lo16, np.maximum(hi16, lo16), rng


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 8])
def test_step_is_correctly_rounded(bits):
    lo, hi, _ = ranges(bits, 3000, bits)
    for l, h in zip(lo, hi):
        d = f32(h - l)
        ref = f32(d / f32(2 ** bits - 1))
        ref = f32(1) if ref == 0 else ref
        assert kivi_step(float(d), bits) == float(ref)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 8])
def test_quotient_is_correctly_rounded(bits):
    L = 2 ** bits - 1
    lo, hi, rng = ranges(bits, 1500, 10 + bits)
    checked = 0
    for l, h in zip(lo, hi):
        step = f32((h - l) / f32(L))
        step = f32(1) if step == 0 else step
        xs = [l, h, f32(l + (h - l) * f32(rng.uniform()))]
        # values whose quotient sits next to a rounding point of t = q + 0.5
        k = f32(rng.integers(0, L + 1)) + f32(0.5)
        near = f32(l + k * step)
        xs += [near, np.nextafter(near, f32(np.inf)), np.nextafter(near, f32(-np.inf))]
        for x in xs:
            a = f32(f32(x) - l)
            ref = f32(a / step)
            if ref != 0 and abs(ref) < np.finfo(np.float32).tiny:
                continue                       # subnormal quotient: its code is 0 either way
            q = quotient(float(a), float(step))
            assert q == float(ref), (float(a), float(step), q, float(ref))
            code = min(max(np.floor(f32(f32(q) + f32(0.5))), 0), L)
            assert code == min(max(np.floor(f32(ref + f32(0.5))), 0), L)
            checked += 1
    assert checked > 8000


def test_uncorrected_product_is_not_enough():
    """The correction step matters: RN(a * RN(1 / step)) alone misses the correctly rounded quotient."""
    rng = np.random.default_rng(5)
    misses = 0
    for _ in range(3000):
        step = f32(np.exp(rng.uniform(-10, 5)))
        a = f32(rng.uniform(0, 16) * step)
        inv = f32(f32(1) / step)
        misses += f32(a * inv) != f32(a / step)
        assert quotient(float(a), float(step)) == float(f32(a / step))
    assert misses > 0


def test_native_sweep(tmp_path):
    """The same arithmetic in C with hardware fmaf over 1.5M ranges x 8 values (tests/division_sweep.c)."""
    import shutil
    import subprocess
    from pathlib import Path
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / "division_sweep"
    src = Path(__file__).with_name("division_sweep.c")
    subprocess.run([cc, "-O2", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe), "1500000"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "code_diff 0" in out.stdout
