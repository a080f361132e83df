"""Key-bias removal (CPU): the oracle's R_t b and the C ABI's checks.

oracle.key_bias_offsets restates reference/mechanism_eval.py:88-97 (bb * cos + rotate_half(bb) * sin with the
model's rotary tables). It is pinned against the rotation it stands for: with the usual RoPE tables
(cos_t = cos(t * f) and sin_t = sin(t * f) for inverse frequencies f, repeated over both halves), R_t b is the
complex product (b_j + i b_{j+d/2}) e^{i t f_j} written back as (real, imaginary) halves; it keeps the norm,
is the identity at position 0, and maps vector v of a token-major cache to token first + v // heads and head
v % heads.
"""
import ctypes

import numpy as np
import pytest

from oracle import pitch_oracle as O


def rope_tables(positions, d, theta=10000.0):
    inv = 1.0 / theta ** (np.arange(0, d, 2) / d)
    ang = np.arange(positions)[:, None] * inv[None, :]
    return (np.concatenate([np.cos(ang)] * 2, 1).astype(np.float32),
            np.concatenate([np.sin(ang)] * 2, 1).astype(np.float32), ang)


@pytest.mark.parametrize("d", [2, 8, 64, 128])
def test_rope_bias_is_the_complex_rotation(d):
    rng = np.random.default_rng(d)
    heads, P = 3, 50
    bias = rng.standard_normal((heads, d)).astype(np.float32)
    cos, sin, ang = rope_tables(P, d)
    o = O.key_bias_offsets(bias, cos, sin, first_position=7, count=heads * 20, heads=heads)
    v = np.arange(heads * 20)
    t, h = 7 + v // heads, v % heads
    z = (bias[h, :d // 2] + 1j * bias[h, d // 2:]).astype(np.complex128) * np.exp(1j * ang[t])
    ref = np.concatenate([z.real, z.imag], 1)
    assert np.allclose(o, ref, rtol=1e-5, atol=1e-5)
    assert np.allclose(np.linalg.norm(o, axis=1), np.linalg.norm(bias[h], axis=1), rtol=1e-5)
    o0 = O.key_bias_offsets(bias, cos, sin, first_position=0, count=heads, heads=heads)
    assert np.array_equal(o0, bias)                                   # R_0 b = b exactly (cos 1, sin 0)


def test_rotate_half():
    x = np.arange(8.0)
    assert O.rotate_half(x).tolist() == [-4, -5, -6, -7, 0, 1, 2, 3]


def test_key_bias_abi_validation(built_library):
    from pitch_amd import _lib
    lib = _lib.load()

    class Host:
        def __init__(self, n):
            self.buf = ctypes.create_string_buffer(max(n, 1))
            self.n = n

        @property
        def p(self):
            return ctypes.cast(self.buf, ctypes.c_void_p)

    cfg = _lib.PitchConfigC(0, 64, 4, 0)
    count, heads = 40, 4
    inp, codes, scales = Host(count * 256), Host(count * 32), Host(count * 4)
    bias, cos, sin = Host(heads * 256), Host(20 * 256), Host(20 * 256)

    def enc(kb):
        return lib.pitch_enqueue_encode_key_bias(ctypes.byref(cfg), ctypes.byref(kb) if kb else None, inp.p, inp.n, 0,
                                                 codes.p, codes.n, 0, scales.p, scales.n, 0, count, None)

    def kb(heads=heads, first=0, table=20 * 256, bias_bytes=heads * 256):
        return _lib.PitchKeyBiasC(bias.p, bias_bytes, cos.p, sin.p, table, first, heads, 0)

    assert enc(None) == _lib.ERR_INVALID_INPUT
    assert enc(kb(heads=0)) == _lib.ERR_INVALID_INPUT
    assert enc(kb(bias_bytes=heads * 256 - 4)) == _lib.ERR_INVALID_INPUT and "key bias" in _lib.last_error()
    assert enc(kb(first=11)) == _lib.ERR_INVALID_INPUT and "positions" in _lib.last_error()   # needs 10 rows
    assert enc(kb(first=10)) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
    assert "positions" not in _lib.last_error()
    rc = lib.pitch_enqueue_decode_key_bias(ctypes.byref(cfg), ctypes.byref(kb(table=9 * 256)), codes.p, codes.n, 0,
                                           scales.p, scales.n, 0, inp.p, inp.n, 0, count, None)
    assert rc == _lib.ERR_INVALID_INPUT and "positions" in _lib.last_error()
