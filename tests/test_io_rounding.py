"""The 16-bit element-type roundings of the oracle and the host-side element-type dispatch (CPU only).

The float16 / bfloat16 entry points are specified as the conversion the reference leaves to its callers
(README.md:97): widen 16-bit inputs to float32 exactly, round float32 outputs to nearest even. The oracle's
conversions are pinned here against two independent library routines, numpy's float16 cast and torch's
bfloat16 cast, on every class of value that decides a rounding: exact values, halfway cases with even and odd
last kept bits, values just above and below a halfway point, the largest finite values and the overflow
threshold, subnormals, signed zeros and infinities, plus a random sweep of bit patterns.
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O


def _special_f32():
    vals = []
    for m in (0x3F800000, 0x3F810000, 0x40490000, 0x7F7F0000, 0x00010000, 0x00000001, 0x0):
        for low in (0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF):
            vals.append(m | low)
            vals.append(m | low | 0x80000000)
    vals += [0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x477FE000, 0x477FF000, 0x477FEFFF, 0x38800000, 0x33800000,
             0x33000000, 0x33000001, 0x387FC000]
    return np.array(vals, dtype=np.uint32).view(np.float32)


def _random_f32(n=400000, seed=5):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    return x[np.isfinite(x)]


def test_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.concatenate([_special_f32(), _random_f32()])
    ours = O.bf16_bits(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.isnan(O.bf16_to_f32(O.bf16_bits(x))).all()


def test_bf16_halfway_cases_round_to_even():
    # 1 + 2^-8 is halfway between 1 and 1 + 2^-7 (kept bit even: down); 1 + 3 * 2^-8 is halfway between
    # 1 + 2^-7 and 1 + 2^-6 (kept bit odd: up)
    x = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)], dtype=np.float32)
    assert O.round_io(x, "bfloat16").tolist() == [1.0, 1 + 2 ** -6, -1.0]


def test_f16_matches_torch_and_numpy():
    torch = pytest.importorskip("torch")
    x = np.concatenate([_special_f32(), _random_f32(seed=6) * np.float32(1e-30)])
    x = x[np.isfinite(x)]
    ours = O.to_io_bits(x, "float16")
    ref = torch.from_numpy(x.copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert O.round_io(np.array([65504.0, 65520.0, 65519.99], np.float32), "float16").tolist() == \
        [65504.0, np.inf, 65504.0]


@pytest.mark.parametrize("io", O.IO_TYPES)
def test_widening_is_exact(io):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(10000).astype(np.float32)
    bits = O.to_io_bits(x, io)
    back = O.from_io_bits(bits, io)
    assert np.array_equal(O.to_io_bits(back, io), bits)       # rounding a representable value is exact
    if io == "float32":
        assert np.array_equal(back, x)
    else:      # round to nearest: relative error at most half an ulp, 2^-11 (float16) or 2^-8 (bfloat16)
        half_ulp = 2.0 ** (-11 if io == "float16" else -8)
        m = np.abs(x) > 1e-4                                  # normal float16 range
        err = np.abs(back.astype(np.float64) - x)[m] / np.abs(x.astype(np.float64))[m]
        assert err.max() <= half_ulp


def test_host_element_type_dispatch():
    torch = pytest.importorskip("torch")
    from pitch_amd import _lib
    from pitch_amd.api import InvalidInput, _io_type
    assert _io_type(torch.empty(1)) == _lib.IO_F32
    assert _io_type(torch.empty(1, dtype=torch.uint8)) == _lib.IO_F32       # raw byte buffers hold float32
    assert _io_type(torch.empty(1, dtype=torch.float16)) == _lib.IO_F16
    assert _io_type(torch.empty(1, dtype=torch.bfloat16)) == _lib.IO_BF16
    assert _io_type(torch.empty(4, dtype=torch.uint8), "bfloat16") == _lib.IO_BF16
    assert _io_type(torch.empty(4, dtype=torch.uint8), torch.float16) == _lib.IO_F16
    with pytest.raises(InvalidInput):
        _io_type(torch.empty(1), "float64")
