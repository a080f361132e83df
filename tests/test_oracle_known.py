"""The CPU oracle against closed forms, library routines, brute force and the reference's known answers.

These pin what the golden vectors pin only implicitly, and each is chosen so that a plausible slip (a dropped
stage, a wrong sign, a transposed index, ties sent the wrong way) fails it:
* FWHT: the Sylvester Hadamard matrix from scipy.linalg.hadamard, H.H = d.I, orthogonality of the rotation;
* PCG hash: an independent implementation on Python integers;
* packing: a brute-force bit-string packer;
* codebooks: ascending, antisymmetric, zero middle edge, and the Lloyd-Max centroid condition against the
  sphere-coordinate density computed in closed form with the regularised incomplete beta function;
* codecs: one-hot error 0.25 at d = 64, b = 2 (RotationWorstCaseTests.swift:33-43), Theorem 1
  (CodecTests.swift:45-52), zero vectors and the tie rule, PolarQuant exact grid points;
* KIVI: constant channel exact, error within half a step (PerChannelTests.swift:102-134).
"""
import math

import numpy as np
import pytest
from scipy.linalg import hadamard
from scipy.special import betainc

from oracle import pitch_oracle as O

DIMS = O.SUPPORTED_DIMS
BITS = list(O.SUPPORTED_BITS)


# ----------------------------------------------------------------------------- rotation
@pytest.mark.parametrize("d", DIMS)
def test_wht_is_sylvester_hadamard(d):
    H = O.wht(np.eye(d))
    assert np.array_equal(H, hadamard(d).astype(np.float64))
    assert np.array_equal(O.wht(H), d * np.eye(d))          # H.H = d.I


@pytest.mark.parametrize("d", [2, 16, 64, 128, 1024])
def test_rotation_is_orthogonal_and_inverted(d):
    rng = np.random.default_rng(d)
    X = rng.standard_normal((8, d))
    Y = O.rotate(X, 7)
    np.testing.assert_allclose(np.linalg.norm(Y, axis=1), np.linalg.norm(X, axis=1), rtol=1e-13)
    np.testing.assert_allclose(O.unrotate(Y, 7), X, rtol=0, atol=1e-12 * np.abs(X).max())
    # the rotation is H.diag(s)/sqrt(d) with H symmetric, so its matrix is that product
    R = O.rotate(np.eye(d), 7).T
    np.testing.assert_allclose(R, hadamard(d) * O.rand_signs(7, d)[None, :] / math.sqrt(d), atol=1e-15)


def _pcg_int(v: int) -> int:
    """PCG-RXS-M-XS 32-bit hash (O'Neill 2014, as a hash in Jarzynski and Olano 2020) on Python integers."""
    state = (v * 747796405 + 2891336453) % 2 ** 32
    word = (((state >> ((state >> 28) + 4)) ^ state) * 277803737) % 2 ** 32
    return ((word >> 22) ^ word) % 2 ** 32


def test_pcg_hash_against_integer_implementation():
    vals = [0, 1, 2, 3, 0x50495443, 0x00C0FFEE, 12345, 2 ** 31, 2 ** 32 - 1, 2 ** 32 - 2] + \
        list(np.random.default_rng(1).integers(0, 2 ** 32, 500, dtype=np.uint64))
    got = O.pcg_hash(np.array(vals, dtype=np.uint64))
    assert [int(g) for g in got] == [_pcg_int(int(v)) for v in vals]


def test_rand_signs_wrap_and_balance():
    # seed + i wraps modulo 2^32
    s = O.rand_signs(2 ** 32 - 2, 4)
    assert list(s) == [1.0 if _pcg_int(v) & 1 else -1.0 for v in (2 ** 32 - 2, 2 ** 32 - 1, 0, 1)]
    s = O.rand_signs(O.DEFAULT_SEED, 1024)
    assert set(np.unique(s)) == {-1.0, 1.0} and abs(s.sum()) < 200


# ----------------------------------------------------------------------------- packing
STRIDES = {(64, 2): 16, (64, 3): 24, (64, 4): 32, (64, 8): 64, (128, 2): 32, (128, 3): 48, (128, 4): 64,
           (128, 8): 128, (1024, 2): 256, (1024, 3): 384, (1024, 4): 512, (1024, 8): 1024, (2, 3): 4,
           (2, 2): 4, (2, 8): 4, (16, 3): 8, (7, 3): 4, (33, 5): 24, (1, 2): 4}


@pytest.mark.parametrize("d,b", sorted(STRIDES))
def test_code_stride(d, b):
    assert O.code_stride_bytes(d, b) == STRIDES[(d, b)]


def _pack_brute(codes, b):
    """Bit string per vector: code i's bits LSB first at positions i*b.., zero-padded to whole words."""
    n, d = codes.shape
    cs = O.code_stride_bytes(d, b)
    out = bytearray()
    for row in codes:
        bits = []
        for c in row:
            bits += [(int(c) >> k) & 1 for k in range(b)]
        bits += [0] * (cs * 8 - len(bits))
        out += bytes(sum(bits[8 * j + k] << k for k in range(8)) for j in range(cs))
    return bytes(out)


@pytest.mark.parametrize("b", BITS)
@pytest.mark.parametrize("d", [1, 2, 7, 16, 33, 64, 128])
def test_pack_against_brute_force(d, b):
    rng = np.random.default_rng(d * 10 + b)
    codes = rng.integers(0, 2 ** b, size=(5, d))
    packed = O.pack_codes(codes, b)
    assert packed == _pack_brute(codes, b)
    assert np.array_equal(O.unpack_codes(packed, 5, d, b), codes)


# ----------------------------------------------------------------------------- codebooks
@pytest.mark.parametrize("d", DIMS)
def test_codebook_invariants_and_centroid_condition(d):
    a = (d - 1) / 2          # a coordinate of a uniform point on S^{d-1} is 2B - 1 with B ~ Beta(a, a)
    for b in BITS:
        c = O.turbo_codebook(d, b)
        c32 = c.astype(np.float32)
        assert c.shape == (2 ** b,) and np.all(np.diff(c) > 0)
        assert np.array_equal(c32, -c32[::-1]), "codebook is not antisymmetric"
        e = O.turbo_edges(d, b)
        assert e[len(e) // 2] == 0.0 and np.all(np.diff(e) > 0)
        assert np.all((e > c[:-1]) & (e < c[1:]))
        # centroid condition: c_k = E[x | e_{k-1} < x < e_k], the mean of the density (1 - x^2)^((d-3)/2)
        lo = (np.concatenate([[-1.0], e]) + 1) / 2
        hi = (np.concatenate([e, [1.0]]) + 1) / 2
        mass = betainc(a, a, hi) - betainc(a, a, lo)
        mean_b = 0.5 * (betainc(a + 1, a, hi) - betainc(a + 1, a, lo)) / mass
        tol = 1e-3 if d == 2 else 1e-5      # the tables come from a gridded Lloyd-Max; d = 2 is singular at +-1
        assert np.abs((2 * mean_b - 1) - c).max() <= tol, (d, b)


# ----------------------------------------------------------------------------- per-vector codecs
def _mean_rel_err(X, Y):
    X = np.asarray(X, np.float64)
    return float((((X - Y) ** 2).sum(1) / (X ** 2).sum(1)).mean())


def test_one_hot_error_is_a_quarter():
    """RotationWorstCaseTests.oneHotExceedsBound: every one-hot at d = 64, b = 2 has error 0.2500.

    FWHT(one-hot)/8 = +-1/8 per coordinate; that lies above the edge 0.1220, so it maps to the centroid
    +-0.18750010 and the error is 64 (0.18750010 - 0.125)^2 = 0.2500008."""
    X = np.eye(64)
    codes, norms = O.turbo_encode(X, 2, O.DEFAULT_SEED)
    assert np.all(norms == 1.0)
    c = O.turbo_codebook(64, 2)
    assert set(np.unique(codes)) <= {0, 3}
    Y = O.turbo_decode(codes, norms, 2, O.DEFAULT_SEED)
    expected = 64 * (c[3] - 0.125) ** 2
    assert expected == pytest.approx(0.2500008, abs=1e-6)
    np.testing.assert_allclose(((X - Y) ** 2).sum(1), expected, rtol=1e-12)


@pytest.mark.parametrize("b", BITS)
def test_turbo_theorem1(b):
    """CodecTests.turboQuantMeetsTheorem1: 4^-b <= E|x - x^|^2/|x|^2 <= (sqrt(3) pi / 2) 4^-b, d = 64."""
    X = np.random.default_rng(100 + b).standard_normal((16384, 64)).astype(np.float32).astype(np.float64)
    codes, norms = O.turbo_encode(X, b)
    e = _mean_rel_err(X, O.turbo_decode(codes, norms.astype(np.float32).astype(np.float64), b))
    lower = 4.0 ** -b
    assert lower <= e <= math.sqrt(3) * math.pi / 2 * lower


@pytest.mark.parametrize("d", [2, 64, 1024])
@pytest.mark.parametrize("b", [2, 3, 8])
def test_zero_vector_and_ties(d, b):
    """Zero in, zero out; u = 0 sits exactly on the middle edge and goes to the lower code (side='left')."""
    X = np.zeros((2, d))
    codes, norms = O.turbo_encode(X, b)
    assert np.all(norms == 0) and np.all(codes == 2 ** (b - 1) - 1)
    assert np.all(O.turbo_decode(codes, norms, b) == 0)
    pc, rmax = O.polar_encode(X, b)
    assert np.all(rmax == 0) and np.all(pc == 0)
    assert np.all(O.polar_decode(pc, rmax, b) == 0)


def edge_straddle_check(d=64, b=4, seed=O.DEFAULT_SEED):
    """Decision edges are the float32 values float32(0.5f * (c[k] + c[k+1])) (reference/pitch_reference.py:99-100),
    not the float64 midpoints: a rotated coordinate placed strictly between the two takes the code that the
    float32 edge gives. Inputs are built by unrotating a chosen unit vector U, so rotate(x / |x|) = U up to
    float64 rounding, far below the gap between the two edge values."""
    c = O.turbo_codebook(d, b)
    e32 = O.turbo_edges(d, b)
    e64 = 0.5 * (c[1:] + c[:-1])
    ks = np.nonzero(e32 != e64)[0]
    assert len(ks) > 0
    rng = np.random.default_rng(d + b)
    for k in ks:
        u0 = 0.5 * (e32[k] + e64[k])
        rest = rng.standard_normal(d - 1)
        U = np.concatenate([[u0], rest / np.linalg.norm(rest) * math.sqrt(1 - u0 * u0)])
        X = O.unrotate(U[None, :], seed) * 3.0
        codes, _ = O.turbo_encode(X, b, seed)
        assert codes[0, 0] == (k + 1 if u0 > e32[k] else k), (d, b, k)


@pytest.mark.parametrize("d,b", [(64, 2), (64, 4), (128, 3), (128, 8), (1024, 4)])
def test_edges_are_float32(d, b):
    edge_straddle_check(d, b)


@pytest.mark.parametrize("d", [2, 16, 128])
@pytest.mark.parametrize("b", [2, 4, 8])
def test_polar_grid_points_are_fixed(d, b):
    """A rotated vector whose pairs sit on the (radius, angle) grid encodes to that grid point and decodes back."""
    rng = np.random.default_rng(d + b)
    RL, N = 2 ** b - 1, 2 ** b
    n, P = 6, d // 2
    jr = rng.integers(0, RL + 1, (n, P))
    jr[:, 0] = RL                                     # the largest radius is rmax
    ka = rng.integers(0, N, (n, P))
    rmax = rng.uniform(0.5, 3.0, n)
    r = jr / RL * rmax[:, None]
    th = ka / N * 2 * np.pi
    Y = np.empty((n, d))
    Y[:, 0::2], Y[:, 1::2] = r * np.cos(th), r * np.sin(th)
    X = O.unrotate(Y, 3)
    codes, got_rmax = O.polar_encode(X, b, 3)
    np.testing.assert_allclose(got_rmax, rmax, rtol=1e-12)
    assert np.array_equal(codes[:, 0::2], jr)
    assert np.array_equal(codes[:, 1::2], np.where(jr == 0, codes[:, 1::2], ka))   # angle of r = 0 is free
    np.testing.assert_allclose(O.polar_decode(codes, got_rmax, b, 3), X, atol=1e-12 * np.abs(X).max())


def test_polar_angle_uses_all_codes():
    """CodecTests.polarAngleCodebookUsesAllCodes (CodecTests.swift:61-64)."""
    X = np.random.default_rng(3).uniform(-1, 1, (64, 64))
    for b in (2, 3, 4):
        codes, _ = O.polar_encode(X, b)
        assert len(np.unique(codes[:, 1::2])) == 2 ** b


# ----------------------------------------------------------------------------- KIVI
def _offset_keys(n, d, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d))
    X[:, :4] += np.array([40.0, -25.0, 18.0, -12.0])[: min(4, d)] + 0.3 * rng.standard_normal((n, min(4, d)))
    return X.astype(np.float32)


def test_channel_constant_channel_is_exact():
    X = np.random.default_rng(5).standard_normal((64, 8)).astype(np.float32)
    X[:, 0] = 1.5
    codes, ranges = O.channel_encode(X, 2)
    assert np.all(O.channel_decode(codes, ranges, 2)[:, 0] == 1.5)


@pytest.mark.parametrize("d", [64, 96, 128])
def test_channel_error_within_half_a_step(d):
    X = _offset_keys(200, d, d)
    b = 4
    codes, ranges = O.channel_encode(X, b)
    Y = O.channel_decode(codes, ranges, b)
    lo = ranges[:, 0].astype(np.float32)
    hi = ranges[:, 1].astype(np.float32)
    g = np.arange(200) // 64
    step = (hi - lo)[g] / np.float32(2 ** b - 1)
    slack = 1e-3 * np.maximum(np.abs(lo), np.abs(hi))[g] + 1e-6
    assert np.all(np.abs(X - Y) <= 0.5 * step + slack)
    assert ranges.shape == (4, 2, d)


def test_channel_rejects_out_of_fp16_range():
    with pytest.raises(ValueError):
        O.channel_encode(np.array([[1.0, 70000.0]], np.float32), 4)
    with pytest.raises(ValueError):
        O.channel_encode(np.array([[1.0, np.nan]], np.float32), 4)


def test_accounting():
    """BatchAPITests.perVectorAccounting and PerChannelTests.storageAccounting."""
    assert O.bits_per_coordinate(64, 3) == 3.5
    assert O.bits_per_coordinate(64, 4) == 4.5
    assert O.channel_bits_per_coordinate(64, 4) == 4.5
    assert O.channel_bits_per_coordinate(128, 4) == 4.5
    assert O.channel_bits_per_coordinate(128, 4, 128) == 4.25
    assert O.channel_group_count(150, 64) == 3


# ----------------------------------------------------------------------------- parity band classifiers
def test_near_boundary_classifiers():
    """The tolerance band of the parity bar: within 1e-6 (relative) of a decision edge or rounding point."""
    e = O.turbo_edges(64, 4)
    k = 11
    U = np.zeros((1, 64))
    U[0, :6] = [e[k], e[k] * (1 + 5e-7), e[k] * (1 + 2e-6), 0.0, 0.5 * (e[k] + e[k + 1]), 1e-9]
    m = O.turbo_near_boundary(U, 4)[0]
    assert list(m[:6]) == [True, True, False, True, False, True]     # 0 and 1e-9 sit on the zero middle edge
    t = np.array([3.0, 3.0 + 2e-6, 3.0 + 1e-5, 2.5, 1e7 + 1.0, 0.5])
    assert list(O._near_integer(t, 1e-6)) == [True, True, False, False, True, False]
    # a polar pair at the origin counts as on a boundary (its angle is decided by signed zeros)
    m = O.polar_near_boundary(np.zeros((1, 4)), 3, 0)
    assert list(m[0]) == [False, True, False, True]           # radius code 0 is clear; the angle of r = 0 is not
    X = O.unrotate(np.array([[0.6, 0.8, 0.3, 0.1]]), 0)
    assert not O.polar_near_boundary(X, 3, 0)[0, 1]           # angle 0.927 rad: 1.68 bins + 0.5, far from a tie
    # KIVI: exact rounding ties are flagged, a value mid-way between ties is not
    Xk = np.array([[0.0], [1.0], [0.5], [0.25]], np.float32)
    mk = O.channel_near_boundary(Xk, 2, 4)[:, 0]
    assert list(mk) == [False, False, True, False]


def test_numpy_min_max_keep_the_last_of_equal_values():
    """The per-channel ranges follow numpy's ndarray.min / max over a group's tokens (pitch_reference.py:150-153),
    which keep the last of equal values: an extreme of zero carries the sign of the channel's last zero. The GPU
    encoders reproduce this rule (tests/test_gpu_signed_zero.py); here it is pinned for the numpy the oracle runs
    on, in 1-D reductions and in the (tokens, channels) axis-0 reductions of a 64-token group."""
    import numpy as np
    # (column, expected sign of the minimum if it is zero, expected sign of the maximum if it is zero)
    cases = [([0.0, -0.0, 1.0], "-", None), ([-0.0, 0.0, 1.0], "+", None), ([1.0, -0.0, 0.0, 2.0], "+", None),
             ([1.0, 0.0, -0.0, 2.0], "-", None), ([-1.0, 0.0, -0.0], None, "-"), ([-1.0, -0.0, 0.0], None, "+"),
             ([0.0, -0.0, 0.0, -0.0], "-", "-"), ([-0.0, 0.0], "+", "+")]
    for col, lo, hi in cases:
        a = np.array(col, np.float32)
        blk = np.empty((64, 9), np.float32)
        blk[:] = 7.0 if lo is not None and hi is None else -7.0   # fillers that do not move a zero extreme
        if lo is not None and hi is not None:
            blk[:] = a[-1]
        blk[:len(a), 5] = a
        if lo is not None and hi is not None:   # all zeros: pad with copies of the last zero
            blk[len(a):, 5] = a[-1]
        for got_lo, got_hi in ((a.min(), a.max()), (blk.min(0)[5], blk.max(0)[5])):
            if lo is not None:
                assert got_lo == 0 and bool(np.signbit(got_lo)) == (lo == "-"), (col, "min")
            if hi is not None:
                assert got_hi == 0 and bool(np.signbit(got_hi)) == (hi == "-"), (col, "max")
