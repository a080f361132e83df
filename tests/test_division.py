"""The per-channel quantiser's guarded quotient (CPU only).

The per-channel encoder (chan_encode_w in pitch_channel.hip) needs t = RN(RN((x - lo) / step) + 0.5) in float32
(reference/pitch_reference.py:157). It first takes t' = RN(RN((x - lo) * RN(1 / step)) + 0.5) and keeps
floor(t') when t' lies at least kKiviGuard = 1e-4 from an integer; otherwise it divides exactly. Emulated here
with numpy float32 arithmetic on the operand ranges the codec sees (fp16-rounded ranges, steps
(hi - lo) / (2^b - 1), values inside and just outside the range):
* |t' - t| stays below a third of the guard;
* whenever the guard accepts, floor(t') equals floor(t), the reference's value;
* the exact division is needed for only a small fraction of values.
"""
import numpy as np
import pytest

f32 = np.float32
GUARD = 1e-4


def operands(bits, n, seed):
    rng = np.random.default_rng(seed)
    lo = rng.standard_normal(n) * np.exp(rng.uniform(-8, 10, n))
    width = np.exp(rng.uniform(-12, 10, n))
    lo16 = np.clip(lo, -65504, 65504).astype(np.float16)
    hi16 = np.clip(lo + width, -65504, 65504).astype(np.float16)
    lo32, hi32 = lo16.astype(f32), hi16.astype(f32)
    step = ((hi32 - lo32) / f32(2 ** bits - 1)).astype(f32)
    step[step == 0] = f32(1)
    x = (lo32 + (hi32 - lo32) * rng.uniform(-0.01, 1.01, n).astype(f32)).astype(f32)
    return (x - lo32).astype(f32), step


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 8])
def test_guarded_quotient(bits):
    a, step = operands(bits, 400000, bits)
    inv = (f32(1) / step).astype(f32)
    t_approx = ((a * inv).astype(f32) + f32(0.5)).astype(f32)
    t_exact = ((a / step).astype(f32) + f32(0.5)).astype(f32)
    assert np.abs(t_approx.astype(np.float64) - t_exact.astype(np.float64)).max() < GUARD / 3
    k = np.floor(t_approx)
    f = t_approx - k
    ok = (f > GUARD) & (f < 1 - GUARD)
    assert np.array_equal(k[ok], np.floor(t_exact)[ok])
    assert ok.mean() > 0.999
