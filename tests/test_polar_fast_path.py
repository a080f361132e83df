"""The PolarQuant encoders' float32 fast paths, emulated on the CPU (CPU only).

pitch_vector.hip decides each radius and angle code from t = value * levels + 0.5 evaluated in float32 and
keeps floor(t) only when t lies at least kPolarGuard = 3e-4 from an integer; otherwise the float64 path
decides. There are two formulations:
* the team encoder (vec_encode; 16-bit inputs and dimensions other than 64 and 128) scales each pair by
  1 / rmax in float64 before rounding it to float32, and takes the angle in turns (angle_turns);
* the staged-stage encoder (vec_encode_hs; float32 inputs at d = 64 and 128) rounds the unscaled pair of the
  unnormalised transform to float32, multiplies the radius by RN((2^b - 1) / rmax) behind a guard of
  (2^b - 1) * 1.2e-6, and takes the angle at b <= 5 from the signs of d_j = fma(mx, -RN(tan_j), mn) against
  the sector boundaries of the first octant (sector_code_tab: guard |d_j| > fma(mx, 2e-6, 1e-36), the code
  looked up in a table indexed by the sign bits of the d_j, of |a| - |c|, of a and of c), above that in sector
  units (angle_sectors: the factor 2^b / (2 pi) folded into the polynomial's coefficients); vectors whose
  largest radius lies outside [1e-15, 1e18] go to the float64 path whole.
This test evaluates the same float32 steps in numpy (fused multiply-adds as one rounding, the reciprocal and
square root correctly rounded, which the hardware's 1-ulp versions can differ from by one ulp) on rotated
K/V-like vectors and checks, for both, that
* the float32 t (and d_j) stays within a third of its guard of the float64 value of the oracle at every bit width,
* every code the guards accept equals the oracle's code (pitch_reference.py:109-121),
* the guards send only a small fraction of pairs to the float64 path.
"""
import importlib.util
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import pitch_oracle as O

ROOT = Path(__file__).resolve().parent.parent
_spec = importlib.util.spec_from_file_location("gen_tables", ROOT / "pitch_amd" / "csrc" / "gen_tables.py")
G = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(G)
GUARD = 3e-4
f32 = np.float32


def _fma32(a, b, c):
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(f32)


def angle_turns(c, a, coef):
    ax, ay = np.abs(a), np.abs(c)
    mx, mn = np.maximum(ax, ay), np.minimum(ax, ay)
    with np.errstate(divide="ignore", invalid="ignore"):
        z = (mn * (f32(1) / mx)).astype(f32)
    s = (z * z).astype(f32)
    p = np.full_like(s, coef[-1])
    for k in coef[-2::-1]:
        p = _fma32(p, s, np.full_like(s, k))
    at = (p * z).astype(f32)
    at = np.where(ay > ax, (f32(np.pi / 2) - at).astype(f32), at)
    at = np.where(a < 0, (f32(np.pi) - at).astype(f32), at)
    turns = (at * f32(1 / (2 * np.pi))).astype(f32)
    return np.where(c < 0, (f32(1) - turns).astype(f32), turns)


def angle_sectors(c, a, coef, b):
    """angle_sectors of pitch_vector.hip: angle_turns * 2^b with 2^b / (2 pi) folded into the coefficients."""
    L = f32(2 ** b)
    kS = f32(2 ** b / (2 * np.pi))
    cs = [f32(k) * kS for k in coef]
    ax, ay = np.abs(a), np.abs(c)
    mx, mn = np.maximum(ax, ay), np.minimum(ax, ay)
    with np.errstate(divide="ignore", invalid="ignore"):
        z = (mn * (f32(1) / mx)).astype(f32)
    s = (z * z).astype(f32)
    p = np.full_like(s, cs[-1])
    for k in cs[-2::-1]:
        p = _fma32(p, s, np.full_like(s, k))
    w = (p * z).astype(f32)
    w = np.where(ay > ax, (f32(0.25) * L - w).astype(f32), w)
    w = np.where(a < 0, (f32(0.5) * L - w).astype(f32), w)
    return np.where(c < 0, (L - w).astype(f32), w)


SECTOR_GUARD = 2e-6


def radius_guard(b):
    return (2 ** b - 1) * 1.2e-6


def sector_table(b):
    """octant_table_build of pitch_vector.hip: the code of each sign-bit index (bit 0 c < 0, bit 1 a < 0, bit 2
    |c| > |a|, bits 3 .. K + 2 d_{K-1} .. d_0 < 0) after the octant reflections of the first-octant count."""
    L, K = 2 ** b, len(G.sector_tans(b))
    tab = np.zeros(1 << (K + 3), np.int64)
    for i in range(len(tab)):
        n = sum(1 for j in range(K) if not (i >> (3 + j)) & 1)
        n = L // 4 - n if (i >> 2) & 1 else n
        n = L // 2 - n if (i >> 1) & 1 else n
        n = L - n if i & 1 else n
        tab[i] = n & (L - 1)
    return tab


def sector_code(c, a, b):
    """sector_code_tab of pitch_vector.hip: (code, accepted, d_j values, mx) of float32 pairs (a, c)."""
    tans = G.sector_tans(b)
    ax, ay = np.abs(a), np.abs(c)
    mx, mn = np.maximum(ax, ay), np.minimum(ax, ay)
    gm = _fma32(mx, np.full_like(mx, f32(SECTOR_GUARD)), np.full_like(mx, f32(1e-36)))
    ok = np.ones(a.shape, bool)
    idx = np.zeros(a.shape, np.int64)
    ds = []
    for t in tans:
        dj = _fma32(mx, np.full_like(mx, -t), mn)
        ds.append(dj)
        idx = 2 * idx + np.signbit(dj)
        ok &= np.abs(dj) > gm
    idx = 2 * idx + np.signbit((ax - ay).astype(f32))
    idx = 2 * idx + np.signbit(a)
    idx = 2 * idx + np.signbit(c)
    return sector_table(b)[idx], ok, ds, mx


def staged_codes(X, b):
    """The staged-stage encoder's float32 decisions for float32 vectors X (as float64): the radius and angle codes
    it computes, whether its guards accept them, and the float32 t values of the radius and the angle."""
    d = X.shape[1]
    L = 2 ** b
    Yu = O.rotate(X, O.DEFAULT_SEED) * math.sqrt(d)  # the transform before the division by sqrt(d)
    a, c = Yu[:, 0::2], Yu[:, 1::2]
    rmax = np.hypot(a, c).max(1, keepdims=True)
    safe = np.where(rmax > 0, rmax, 1.0)
    af, cf = a.astype(f32), c.astype(f32)
    with np.errstate(over="ignore", invalid="ignore"):
        rf = np.sqrt(_fma32(af, af, (cf * cf).astype(f32))).astype(f32)
        sr = ((L - 1) / safe).astype(f32)
        tr = _fma32(rf, np.broadcast_to(sr, rf.shape), np.full_like(rf, f32(0.5)))
        gr = radius_guard(b)
        fr = tr - np.floor(tr)
        ok = (rmax >= 1e-15) & (rmax <= 1e18) & (fr > gr) & (fr < 1 - gr)
        if b in G.SECTOR_BITS:
            ac, oka, _, _ = sector_code(cf, af, b)
            ta = None
            ok &= oka
        else:
            ta = (angle_sectors(cf, af, G.atan_poly(G.ATAN_DEG[b]), b) + f32(0.5)).astype(f32)
            fa = ta - np.floor(ta)
            ok &= (fa > GUARD) & (fa < 1 - GUARD)
            ac = np.floor(np.nan_to_num(ta)).astype(np.int64) & (L - 1)
        rc = np.floor(np.nan_to_num(tr, posinf=0.0)).astype(np.int64)
    return rc, ac, ok, tr, ta


@pytest.mark.parametrize("b", list(G.SECTOR_BITS))
def test_sector_code_error_budget(b):
    """Full circle at several magnitudes: each computed d_j lies within a third of the guard (2e-6 mx) of the
    float64 value of mn - mx tan((j - 1/2) 2 pi / 2^b) for the same float32 pair, and the accepted codes equal
    floor(atan2 / (2 pi) * 2^b + 0.5) mod 2^b in float64 (pitch_reference.py:114-117)."""
    th = np.linspace(-math.pi, math.pi, 200001)
    L = 2 ** b
    for mag in (1e-35, 1e-33, 1e-29, 1e-3, 1.0, 7.5e4, 1e29):
        a, c = (mag * np.cos(th)).astype(f32), (mag * np.sin(th)).astype(f32)
        code, ok, ds, mx = sector_code(c, a, b)
        a64, c64 = a.astype(np.float64), c.astype(np.float64)
        mx64 = np.maximum(np.abs(a64), np.abs(c64))
        mn64 = np.minimum(np.abs(a64), np.abs(c64))
        k = np.arange(1, len(ds) + 1)
        for j, dj in zip(k, ds):
            exact = mn64 - mx64 * np.tan((j - 0.5) * 2 * np.pi / L)
            assert np.abs(dj.astype(np.float64) - exact).max() < SECTOR_GUARD / 3 * mx64.max(), (b, mag, j)
        th64 = np.mod(np.arctan2(c64, a64), 2 * np.pi)
        ref = np.floor(th64 / (2 * np.pi) * L + 0.5).astype(np.int64) & (L - 1)
        assert np.array_equal(code[ok], ref[ok]), (b, mag)
        # the guard's 1e-36 floor widens it below mx of about 1e-31
        assert ok.mean() > (0.999 if mag > 1e-32 else (0.99 if mag > 1e-34 else 0.05)), (b, mag, ok.mean())
    # the origin and pairs below 1e-36 are left to the float64 path
    z = np.array([0.0, -0.0, 1e-37, 0.0], f32)
    _, ok, _, _ = sector_code(z, z[::-1].copy(), b)
    assert not ok.any()


@pytest.mark.parametrize("d", [64, 128])
def test_staged_fast_path_matches_oracle(d):
    """The staged-stage encoder's formulation, on the unnormalised transform as the kernel holds it."""
    rng = np.random.default_rng(100 + d)
    X = rng.standard_t(5, size=(6000, d)) * np.exp(rng.uniform(-2, 3, size=(6000, 1))) + rng.normal(0, 2, (1, d))
    X = X.astype(np.float32).astype(np.float64)
    Yu = O.rotate(X, O.DEFAULT_SEED) * math.sqrt(d)
    ru = np.hypot(Yu[:, 0::2], Yu[:, 1::2])
    safe = ru.max(1, keepdims=True)
    _, theta = O.polar_parts(X)
    for b in range(2, 9):
        L = 2 ** b
        rc, ac, ok, tr, ta = staged_codes(X, b)
        tr_exact = ru / safe * (L - 1) + 0.5
        assert np.abs(tr - tr_exact).max() < radius_guard(b) / 3, b
        assert tr.max() < L - 0.5 + 1e-4, b  # the radius code needs no clip
        if ta is not None:
            da = np.abs(ta - (theta / (2 * np.pi) * L + 0.5))
            assert np.minimum(da, np.abs(da - L)).max() < GUARD / 3, b
        codes, _ = O.polar_encode(X, b)
        assert np.array_equal(rc[ok], codes[:, 0::2][ok]), b
        assert np.array_equal(ac[ok], codes[:, 1::2][ok]), b
        assert ok.mean() > (0.9999 if b in G.SECTOR_BITS else 0.998), (b, ok.mean())


@pytest.mark.parametrize("b", [2, 4, 8])
def test_staged_fast_path_at_extreme_magnitudes(b):
    """Vectors scaled from 1e-33 to 1e19: every code the staged formulation accepts equals the oracle's. Below a
    largest radius of about 1e-18 the float32 squares of the unscaled pairs lose their precision (near 1e-25 they
    underflow and every radius would read 0), which the [1e-15, 1e18] range check keeps off the fast path;
    above about 1.8e19 they overflow."""
    rng = np.random.default_rng(b)
    d = 128
    G0 = rng.standard_normal((300, d))
    for scale in (1e-33, 1e-29, 1e-25, 1e-21, 1e-19, 1e-17, 1e-16, 1e-3, 1.0, 1e9, 1e16, 1e17, 1e19):
        X = (G0 * scale).astype(np.float32).astype(np.float64)
        rc, ac, ok, _, _ = staged_codes(X, b)
        codes, _ = O.polar_encode(X, b)
        assert np.array_equal(rc[ok], codes[:, 0::2][ok]), (b, scale)
        assert np.array_equal(ac[ok], codes[:, 1::2][ok]), (b, scale)
        if 1e-13 < scale < 1e16:
            assert ok.mean() > 0.99, (b, scale, ok.mean())
    # the range check is what keeps the tiny vectors right: without it their radius codes are wrong
    X = (G0 * 1e-25).astype(np.float32).astype(np.float64)
    rc, _, _, tr, _ = staged_codes(X, b)
    codes, _ = O.polar_encode(X, b)
    assert (rc != codes[:, 0::2]).mean() > 0.5


@pytest.mark.parametrize("b", range(2, 9))
def test_sector_angle_error_budget(b):
    """Full circle: the emulated sector-unit angle keeps t = w + 0.5 within 1e-4 of the exact t."""
    coef = G.atan_poly(G.ATAN_DEG[b])
    th = np.linspace(-math.pi, math.pi, 400001)
    a, c = np.cos(th).astype(f32), np.sin(th).astype(f32)
    w = angle_sectors(c, a, coef, b).astype(np.float64)
    ref = np.mod(np.arctan2(c.astype(np.float64), a.astype(np.float64)), 2 * np.pi) / (2 * np.pi) * 2 ** b
    err = np.abs(w - ref)
    err = np.minimum(err, 2 ** b - err)
    assert err.max() < 1e-4


@pytest.mark.parametrize("d", [16, 64, 128])
def test_fast_path_matches_oracle(d):
    rng = np.random.default_rng(d)
    X = rng.standard_t(5, size=(6000, d)) * np.exp(rng.uniform(-2, 3, size=(6000, 1))) + rng.normal(0, 2, (1, d))
    X = X.astype(np.float32).astype(np.float64)
    Y = O.rotate(X, O.DEFAULT_SEED)
    a, c = Y[:, 0::2], Y[:, 1::2]
    r, theta = O.polar_parts(X)
    rmax = r.max(1, keepdims=True)
    inv = 1.0 / np.where(rmax > 0, rmax, 1.0)
    af, cf = (a * inv).astype(f32), (c * inv).astype(f32)
    rf = np.sqrt(_fma32(af, af, (cf * cf).astype(f32))).astype(f32)
    for b in range(2, 9):
        L = 2 ** b
        turns = angle_turns(cf, af, G.atan_poly(G.ATAN_DEG[b]))
        tr = _fma32(rf, np.full_like(rf, f32(L - 1)), np.full_like(rf, f32(0.5)))
        ta = _fma32(turns, np.full_like(turns, f32(L)), np.full_like(turns, f32(0.5)))
        tr_exact = r * inv * (L - 1) + 0.5
        ta_exact = theta / (2 * np.pi) * L + 0.5
        # the angle's t is compared modulo L (a direction just below 2 pi wraps to code 0)
        da = np.abs(ta - ta_exact)
        da = np.minimum(da, np.abs(da - L))
        assert np.abs(tr - tr_exact).max() < GUARD / 3, b
        assert da.max() < GUARD / 3, b
        fr, fa = tr - np.floor(tr), ta - np.floor(ta)
        ok = (r > 0) & (fr > GUARD) & (fr < 1 - GUARD) & (fa > GUARD) & (fa < 1 - GUARD)
        codes, _ = O.polar_encode(X, b)
        rc = np.minimum(np.floor(tr), L - 1).astype(np.int64)
        ac = np.floor(ta).astype(np.int64) & (L - 1)
        assert np.array_equal(rc[ok], codes[:, 0::2][ok]), b
        assert np.array_equal(ac[ok], codes[:, 1::2][ok]), b
        assert ok.mean() > 0.99, (b, ok.mean())


@pytest.mark.parametrize("b", range(2, 9))
def test_angle_error_budget(b):
    """Full circle: the emulated float32 angle keeps t = turns * 2^b + 0.5 within 1e-4 of the exact t."""
    coef = G.atan_poly(G.ATAN_DEG[b])
    th = np.linspace(-math.pi, math.pi, 400001)
    a, c = np.cos(th).astype(f32), np.sin(th).astype(f32)
    turns = angle_turns(c, a, coef).astype(np.float64)
    ref = np.mod(np.arctan2(c.astype(np.float64), a.astype(np.float64)), 2 * np.pi) / (2 * np.pi)
    err = np.abs(turns - ref)
    err = np.minimum(err, 1 - err)
    assert err.max() * 2 ** b < 1e-4
