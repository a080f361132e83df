"""The operator contract on the GPU: offsets, ownership, batching, determinism, validation, accuracy.

Mirrors the reference's device tests through the same calls:
* BatchAPITests (Tests/PITCHTests/BatchAPITests.swift:21-116): batching is exact, append/slice, decode into a
  caller buffer at an offset with sentinels either side, the GPU-resident pipeline equals the array API,
  undersized and misaligned buffers are refused;
* CodecBehaviourTests and CodecAccuracyTests (Tests/PITCHTests/CodecTests.swift:27-157): zero vector, scale
  invariance, seeds, invalid inputs, the largest allowed magnitude, accuracy thresholds, Theorem 1, error
  falling with bits, PolarQuant angle codes, d in {2, 1024};
* RotationWorstCaseTests (RotationWorstCaseTests.swift:33-62): one-hot error 0.25, outlier channel;
* PerChannelTests (PerChannelTests.swift:100-212): half-step bound, constant channel, partial final group,
  per-group enqueue at offsets equals the whole block, beats TurboQuant on offset keys;
plus parity with the CPU oracle at every supported dimension (per-vector codes to the counted near-boundary
band, KIVI bit-exact).
"""
import math

import numpy as np
import pytest

from oracle import pitch_oracle as O
from test_gpu_parity import band_mask, check_codes, check_scales, max_rel_diff, mean_rel_err, REL_L2_BAR

pytestmark = pytest.mark.gpu
METHODS = ["turboQuant", "polarQuant"]


def gaussian(n, d, seed):
    return np.random.default_rng(seed).standard_normal((n, d)).astype(np.float32)


def uniform(n, d, seed):
    return np.random.default_rng(seed).uniform(-1, 1, (n, d)).astype(np.float32)


def offset_keys(n, d, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d))
    X[:, :4] += np.array([40.0, -25.0, 18.0, -12.0]) + 0.3 * rng.standard_normal((n, 4))
    return X.astype(np.float32)


# ----------------------------------------------------------------------------- batching and buffers
@pytest.mark.parametrize("method", METHODS)
def test_batch_equals_individual_encodes(q, method):
    X = gaussian(16, 128, 10)
    batch = q.encode(X.reshape(-1), dim=128, bits=3, method=method)
    for i in range(16):
        assert batch.vectors(range(i, i + 1)) == q.encode(X[i], bits=3, method=method)


@pytest.mark.parametrize("method", METHODS)
def test_append_and_slice_round_trip(q, method):
    whole = q.encode(gaussian(10, 64, 11).reshape(-1), dim=64, bits=4, method=method)
    built = whole.vectors(range(0, 3))
    built.append(whole.vectors(range(3, 10)))
    assert built == whole and built.count == 10


@pytest.mark.parametrize("method", METHODS)
def test_decode_into_caller_buffer_at_offset(q, method):
    import torch
    d, n, off = 256, 4, 32
    batch = q.encode(gaussian(n, d, 14).reshape(-1), dim=d, bits=4, method=method)
    expected = q.decode(batch)
    buf = torch.full((off + n * d + off,), -12345.0, dtype=torch.float32, device=q.device)
    q.decode_into(batch, buf, offset=off * 4)
    got = buf.cpu().numpy()
    assert np.array_equal(got[off:off + n * d], expected)
    assert np.all(got[:off] == -12345.0) and np.all(got[off + n * d:] == -12345.0)


@pytest.mark.parametrize("method", METHODS)
def test_gpu_resident_pipeline_matches_array_api(q, method):
    import torch
    import pitch_amd as P
    d, n = 128, 32
    cfg = q.config(method, d, 4)
    X = gaussian(n, d, 15)
    s = torch.cuda.Stream(q.device)
    x = torch.from_numpy(X.reshape(-1)).to(q.device)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    scales = torch.empty(n, dtype=torch.float32, device=q.device)
    out = torch.empty(n * d, dtype=torch.float32, device=q.device)
    torch.cuda.synchronize()
    q.enqueueEncode(x, codes, scales, n, cfg, stream=s)
    q.enqueueDecode(codes, scales, out, n, cfg, stream=s)
    s.synchronize()
    assert np.array_equal(out.cpu().numpy(), q.decode(q.encode(X.reshape(-1), config=cfg)))
    assert isinstance(cfg, P.QuantConfig)


@pytest.mark.parametrize("method", METHODS)
def test_enqueue_at_offsets_into_a_whole_cache(q, method):
    """Append-style encode (12 vectors per token at codesOffset = t * 12 * codeStride)."""
    import torch
    d, heads, T = 64, 12, 9
    cfg = q.config(method, d, 4)
    X = gaussian(T * heads, d, 16)
    x = torch.from_numpy(X.reshape(-1)).to(q.device)
    codes = torch.zeros(T * heads * cfg.codeStride + 64, dtype=torch.uint8, device=q.device)
    scales = torch.zeros(T * heads + 16, dtype=torch.float32, device=q.device)
    for t in range(T):
        q.enqueueEncode(x, codes, scales, heads, cfg, inputOffset=t * heads * d * 4,
                        codesOffset=t * heads * cfg.codeStride, scalesOffset=t * heads * 4)
    torch.cuda.synchronize()
    whole = q.encode(X.reshape(-1), config=cfg)
    c = codes.cpu().numpy()
    assert c[:T * heads * cfg.codeStride].tobytes() == whole.codes and not c[T * heads * cfg.codeStride:].any()
    sc = scales.cpu().numpy()
    assert np.array_equal(sc[:T * heads], whole.scales) and not sc[T * heads:].any()


@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("d", [2, 16, 64, 128])
def test_word_aligned_offsets(q, method, d):
    """Offsets need only be multiples of 4 bytes (Codec.swift:37-47): 4, 8 and 12 modulo 16 all work."""
    import torch
    n = 70
    cfg = q.config(method, d, 3)
    X = gaussian(n, d, 17 + d)
    whole = q.encode(X.reshape(-1), config=cfg)
    expected = q.decode(whole)
    for off in (4, 8, 12):
        x = torch.zeros(off // 4 + n * d, dtype=torch.float32, device=q.device)
        x[off // 4:] = torch.from_numpy(X.reshape(-1)).to(q.device)
        codes = torch.zeros(off + n * cfg.codeStride, dtype=torch.uint8, device=q.device)
        scales = torch.zeros(off // 4 + n, dtype=torch.float32, device=q.device)
        out = torch.full((off // 4 + n * d + 3,), 7.0, dtype=torch.float32, device=q.device)
        q.enqueueEncode(x, codes, scales, n, cfg, inputOffset=off, codesOffset=off, scalesOffset=off)
        q.enqueueDecode(codes, scales, out, n, cfg, codesOffset=off, scalesOffset=off, outputOffset=off)
        torch.cuda.synchronize()
        assert codes.cpu().numpy()[off:].tobytes() == whole.codes
        assert np.array_equal(scales.cpu().numpy()[off // 4:], whole.scales)
        o = out.cpu().numpy()
        assert np.array_equal(o[off // 4:off // 4 + n * d], expected)
        assert np.all(o[:off // 4] == 7.0) and np.all(o[off // 4 + n * d:] == 7.0)


def test_reciprocal_selftest(q):
    """The per-channel encoder forms RN(1 / step) as v_rcp_f32 plus one Newton step; pitch_selftest_reciprocal
    checks on this device that this equals the correctly rounded reciprocal for every positive normal float
    below 2^126 (steps are at most 131008 / 3)."""
    import ctypes
    from pitch_amd import _lib
    n = ctypes.c_uint64(12345)
    assert _lib.load().pitch_selftest_reciprocal(ctypes.byref(n)) == 0, _lib.last_error()
    assert n.value == 0, f"{n.value} floats whose reciprocal is not correctly rounded"


def test_channel_word_aligned_offsets(q):
    import torch
    d, n = 36, 100
    cfg = q.channelConfig(d, 4, 16)
    X = offset_keys(n, d, 21)
    whole = q.encodePerChannel(X.reshape(-1), config=cfg)
    expected = q.decodePerChannel(whole)
    for off in (4, 8, 12):
        x = torch.zeros(off // 4 + n * d, dtype=torch.float32, device=q.device)
        x[off // 4:] = torch.from_numpy(X.reshape(-1)).to(q.device)
        codes = torch.zeros(off + n * cfg.codeStride, dtype=torch.uint8, device=q.device)
        ranges = torch.zeros(off // 2 + cfg.groupCount(n) * cfg.rangeStride // 2, dtype=torch.float16,
                             device=q.device)
        out = torch.full((off // 4 + n * d + 3,), 7.0, dtype=torch.float32, device=q.device)
        q.enqueuePerChannelEncode(x, codes, ranges, n, cfg, inputOffset=off, codesOffset=off, rangesOffset=off)
        q.enqueuePerChannelDecode(codes, ranges, out, n, cfg, codesOffset=off, rangesOffset=off, outputOffset=off)
        torch.cuda.synchronize()
        assert codes.cpu().numpy()[off:].tobytes() == whole.codes
        assert np.array_equal(ranges.cpu().numpy().view(np.uint16)[off // 2:], whole.ranges)
        o = out.cpu().numpy()
        assert np.array_equal(o[off // 4:off // 4 + n * d], expected)
        assert np.all(o[:off // 4] == 7.0) and np.all(o[off // 4 + n * d:] == 7.0)


def test_enqueue_rejects_undersized_and_misaligned(q):
    import torch
    import pitch_amd as P
    cfg = q.config("turboQuant", 64, 4)
    dev = q.device
    x = torch.ones(64 * 4, device=dev)
    with pytest.raises(P.InvalidInput):
        q.enqueueEncode(x, torch.empty(cfg.codeStride * 3, dtype=torch.uint8, device=dev),
                        torch.empty(4, device=dev), 4, cfg)
    pc = q.config("polarQuant", 64, 4)
    with pytest.raises(P.InvalidInput):
        q.enqueueDecode(torch.empty(1024, dtype=torch.uint8, device=dev), torch.empty(16, device=dev),
                        torch.empty(1024, device=dev), 1, pc, codesOffset=2)
    with pytest.raises(P.InvalidInput):
        q.enqueueEncode(x.cpu(), torch.empty(128, dtype=torch.uint8, device=dev), torch.empty(4, device=dev), 1, cfg)
    torch.cuda.synchronize()


# ----------------------------------------------------------------------------- behaviour
@pytest.mark.parametrize("method", METHODS)
def test_zero_vector_decodes_to_zero(q, method):
    out = q.decode(q.encode(np.zeros(64, np.float32), bits=4, method=method))
    assert np.all(out == 0)


@pytest.mark.parametrize("method", METHODS)
def test_scale_invariance(q, method):
    X = gaussian(4, 128, 4).reshape(-1)
    a = q.decode(q.encode(X, dim=128, bits=4, method=method))
    b = q.decode(q.encode(X * 1000, dim=128, bits=4, method=method))
    assert max_rel_diff(b / 1000, a, 128) < 1e-4


@pytest.mark.parametrize("method", METHODS)
def test_seeds(q, method):
    import pitch_amd as P
    X = uniform(8, 256, 5).reshape(-1)
    assert q.encode(X, dim=256, bits=4, method=method, seed=42) == q.encode(X, dim=256, bits=4, method=method, seed=42)
    assert q.encode(X, dim=256, bits=4, method=method, seed=1).codes != \
        q.encode(X, dim=256, bits=4, method=method, seed=2).codes
    x1 = uniform(1, 64, 7).reshape(-1)
    assert q.encode(x1, bits=4, method="turboQuant").config.seed == P.DEFAULT_SEED
    assert P.PITCH(seed=7, device=q.device).encode(x1, bits=4, method="turboQuant").config.seed == 7
    assert q.encode(x1, bits=4, method="turboQuant", seed=99).config.seed == 99


def test_invalid_inputs_through_the_codec(q):
    import pitch_amd as P
    for dim in (0, 1, 3, 100, 2048):
        with pytest.raises(P.PITCHError):
            q.encode(np.ones(max(dim, 1), np.float32), dim=dim, bits=4, method="turboQuant")
    for bits in (0, 1, 9, 16):
        with pytest.raises(P.InvalidBitWidth):
            q.encode(np.ones(64, np.float32), bits=bits, method="polarQuant")
    with pytest.raises(P.InvalidInput):
        q.encode(np.ones(0, np.float32), dim=64, bits=4, method="turboQuant")
    with pytest.raises(P.InvalidInput):
        q.encode(np.ones(100, np.float32), dim=64, bits=4, method="turboQuant")
    for bad in (np.nan, np.inf, -np.inf, 1e30, -1e18):
        for pos in (0, 37, 4095):
            x = np.full(4096, 0.5, np.float32)
            x[pos] = bad
            with pytest.raises(P.InvalidInput):
                q.encode(x, dim=64, bits=4, method="turboQuant")


@pytest.mark.parametrize("method", METHODS)
def test_largest_allowed_magnitude_round_trips(q, method):
    x = np.full(1024, 1e17, np.float32)
    out = q.decode(q.encode(x, bits=8, method=method))
    assert np.all(np.isfinite(out))
    assert mean_rel_err(x, out, 1024) < 0.01


ROUND_TRIP = [("turboQuant", 2, 0.14), ("turboQuant", 3, 0.045), ("turboQuant", 4, 0.013),
              ("turboQuant", 8, 1.5e-4), ("polarQuant", 2, 0.30), ("polarQuant", 3, 0.075),
              ("polarQuant", 4, 0.02), ("polarQuant", 8, 7.5e-5)]


@pytest.mark.parametrize("method,bits,threshold", ROUND_TRIP)
@pytest.mark.parametrize("d", [64, 512])
def test_round_trip_accuracy(q, method, bits, threshold, d):
    """CodecAccuracyTests.roundTrip: mean relative error over 64 U[-1,1] vectors below the threshold."""
    X = uniform(64, d, 1000 + bits).reshape(-1)
    assert mean_rel_err(X, q.decode(q.encode(X, dim=d, bits=bits, method=method)), d) < threshold


@pytest.mark.parametrize("bits", range(2, 9))
def test_turbo_theorem1(q, bits):
    X = gaussian(16384, 64, 200 + bits).reshape(-1)
    e = mean_rel_err(X, q.decode(q.encode(X, dim=64, bits=bits, method="turboQuant")), 64)
    lower = 4.0 ** -bits
    assert lower <= e <= math.sqrt(3) * math.pi / 2 * lower


@pytest.mark.parametrize("method", METHODS)
def test_error_falls_with_bits(q, method):
    X = uniform(64, 256, 9).reshape(-1)
    e = [mean_rel_err(X, q.decode(q.encode(X, dim=256, bits=b, method=method)), 256) for b in (2, 3, 4, 8)]
    assert e[0] > 2 * e[1] and e[1] > 2 * e[2] and e[2] > 50 * e[3]


def test_polar_angle_codes_all_used(q):
    X = uniform(64, 64, 3).reshape(-1)
    for b in (2, 3, 4):
        batch = q.encode(X, dim=64, bits=b, method="polarQuant")
        codes = O.unpack_codes(batch.codes, 64, 64, b)
        assert len(np.unique(codes[:, 1::2])) == 2 ** b


def test_one_hot_error_is_a_quarter(q):
    import pitch_amd as P
    p = P.PITCH(device=q.device)
    X = np.eye(64, dtype=np.float32).reshape(-1)
    err = mean_rel_err(X, p.decode(p.encode(X, dim=64, bits=2, method="turboQuant")), 64)
    assert abs(err - 0.25) < 1e-3


def test_outlier_channel_within_bound(q):
    rng = np.random.default_rng(77)
    X = rng.standard_normal((2048, 64)).astype(np.float32)
    X[np.arange(2048), rng.integers(0, 64, 2048)] *= 30
    err = mean_rel_err(X, q.decode(q.encode(X.reshape(-1), dim=64, bits=2, method="turboQuant")), 64)
    assert err <= math.sqrt(3) * math.pi / 2 / 16


# ----------------------------------------------------------------------------- parity at every dimension
@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("d", [2, 4, 8, 16, 32, 256, 512, 1024])
@pytest.mark.parametrize("bits", [2, 3, 5, 8])
def test_every_dimension_against_oracle(q, method, d, bits):
    import pitch_amd as P
    n = 64 if d >= 512 else 300
    rng = np.random.default_rng(d * 10 + bits)
    X = (rng.standard_t(5, size=(n, d)) * np.exp(rng.uniform(-1, 1.5, size=(n, 1)))).astype(np.float32)
    cfg = P.QuantConfig(method, d, bits, 0x00C0FFEE)
    ours = q.encode(X.reshape(-1), config=cfg)
    codes, scales = O.ENCODERS[method](X.astype(np.float64), bits, 0x00C0FFEE)
    check_codes(method, X, bits, 0x00C0FFEE, ours.codes, O.pack_codes(codes, bits), f"{method} d{d} b{bits}")
    check_scales(ours.scales, np.asarray(scales, np.float32), "scales")
    s32 = np.asarray(scales, np.float32)
    recon = O.DECODERS[method](codes, s32.astype(np.float64), bits, 0x00C0FFEE)
    dec = q.decode(P.CompressedBatch(cfg, O.pack_codes(codes, bits), s32))
    assert max_rel_diff(dec, recon, d) < REL_L2_BAR


@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("d", [128, 256, 1024])
@pytest.mark.parametrize("bits", [3, 6])
def test_extreme_vectors_against_oracle(q, method, d, bits):
    """Zero vectors, vectors at the largest allowed magnitude, tiny vectors (PolarQuant's rmax far below 1e-30 in
    the unnormalised transform), a single huge coordinate among small ones and ordinary vectors, in one call: codes
    equal the oracle's except at near-boundary coordinates, scales within one ulp, decodes finite. A constant
    vector rotates onto a few distinct values, many of them zeros on TurboQuant's middle edge, exact here and
    float64 noise of either sign in the specification's divide-first order (pitch_reference.py:96-101): a dozen or
    more in-band differences at once, so no cap on their count here, unlike the random inputs of check_codes."""
    import pitch_amd as P
    rng = np.random.default_rng(d + bits)
    rows = [np.zeros(d), np.full(d, 1e17), rng.standard_normal(d) * 1e-33, rng.standard_normal(d) * 1e-17,
            np.where(np.arange(d) == 5, 1e16, rng.standard_normal(d) * 1e-3), -np.full(d, 1e17)]
    rows += list(rng.standard_normal((10, d)) * np.exp(rng.uniform(-3, 3, (10, 1))))
    X = np.asarray(rows, np.float32)
    n = len(X)
    cfg = P.QuantConfig(method, d, bits, 0x5EED)
    ours = q.encode(X.reshape(-1), config=cfg)
    codes, scales = O.ENCODERS[method](X.astype(np.float64), bits, 0x5EED)
    diff = O.unpack_codes(ours.codes, n, d, bits) != O.unpack_codes(O.pack_codes(codes, bits), n, d, bits)
    band = band_mask(method, X, None, bits, 0x5EED)
    assert not (diff & ~band).any(), f"{method} d{d} b{bits}: codes differ away from any boundary"
    assert not diff[2:5].any() and not diff[6:].any(), "a non-constant vector differs in the band"
    check_scales(ours.scales, np.asarray(scales, np.float32), "scales")
    assert np.all(np.isfinite(q.decode(ours)))


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_polar_magnitudes_against_oracle(q, d, bits):
    """PolarQuant vectors scaled from 1e-29 up to the largest allowed magnitude (1e17, PITCH.swift:172-181), five
    of each scale, in one call: codes equal the oracle's except at near-boundary coordinates, scales within one
    ulp. The staged encoders (float32 input at d = 64 and 128; d >= 256) decide codes in float32 on the
    unnormalised pairs, whose squared radius loses its precision below a largest radius of about 1e-18 (near
    1e-25 it underflows to 0 and every radius would read code 0) and overflows above about 1.8e19; vectors
    outside the fast path's range take the float64 path."""
    import pitch_amd as P
    rng = np.random.default_rng(31 * d + bits)
    scales_in = np.repeat([1e-29, 1e-25, 1e-21, 1e-19, 1e-17, 1e-16, 1e-3, 1e15, 3e16], 5)
    X = np.clip(rng.standard_normal((len(scales_in), d)) * scales_in[:, None], -1e17, 1e17).astype(np.float32)
    n = len(X)
    cfg = P.QuantConfig("polarQuant", d, bits, 0x5EED)
    print(f"polar magnitudes d{d} b{bits}", flush=True)
    ours = q.encode(X.reshape(-1), config=cfg)
    codes, scales = O.polar_encode(X.astype(np.float64), bits, 0x5EED)
    diff = O.unpack_codes(ours.codes, n, d, bits) != O.unpack_codes(O.pack_codes(codes, bits), n, d, bits)
    band = band_mask("polarQuant", X, None, bits, 0x5EED)
    bad = (diff & ~band).any(1)
    assert not bad.any(), f"d{d} b{bits}: codes differ away from any boundary at scales {sorted(set(scales_in[bad]))}"
    check_scales(ours.scales, np.asarray(scales, np.float32), "scales")


# ----------------------------------------------------------------------------- per-channel
@pytest.mark.parametrize("d", [64, 96, 128])
def test_channel_error_within_half_a_step(q, d):
    X = offset_keys(200, d, d)
    block = q.encodePerChannel(X.reshape(-1), dim=d, bits=4)
    Y = q.decodePerChannel(block).reshape(200, d)
    for t in range(0, 200, 7):
        g = t // 64
        for ch in range(d):
            lo, hi = block.range(g, ch)
            step = (hi - lo) / 15
            assert abs(X[t, ch] - Y[t, ch]) <= 0.5 * step + 1e-3 * max(abs(lo), abs(hi)) + 1e-6


def test_channel_beats_turbo_on_offset_keys(q):
    X = offset_keys(256, 64, 3).reshape(-1)
    ch = q.decodePerChannel(q.encodePerChannel(X, dim=64, bits=4))
    tq = q.decode(q.encode(X, dim=64, bits=4, method="turboQuant"))
    assert ((X - ch) ** 2).mean() < 0.5 * ((X - tq) ** 2).mean()


def test_channel_constant_channel_and_partial_group(q):
    X = gaussian(64, 8, 5)
    X[:, 0] = 1.5
    y = q.decodePerChannel(q.encodePerChannel(X.reshape(-1), dim=8, bits=2)).reshape(64, 8)
    assert np.all(y[:, 0] == 1.5)
    block = q.encodePerChannel(offset_keys(150, 64, 9).reshape(-1), dim=64, bits=4)
    assert block.count == 150 and block.groupCount == 3 and block.ranges.shape[0] == 3 * 2 * 64


def test_channel_groupwise_enqueue_matches_whole_block(q):
    import torch
    d, n = 64, 150
    cfg = q.channelConfig(d, 4)
    X = offset_keys(n, d, 11)
    dev = q.device
    x = torch.from_numpy(X.reshape(-1)).to(dev)
    groups = cfg.groupCount(n)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    ranges = torch.empty(groups * cfg.rangeStride // 2, dtype=torch.float16, device=dev)
    out = torch.empty(n * d, dtype=torch.float32, device=dev)
    for g in range(groups):
        first = g * cfg.groupSize
        m = min(cfg.groupSize, n - first)
        q.enqueuePerChannelEncode(x, codes, ranges, m, cfg, inputOffset=first * d * 4,
                                  codesOffset=first * cfg.codeStride, rangesOffset=g * cfg.rangeStride)
    q.enqueuePerChannelDecode(codes, ranges, out, n, cfg)
    torch.cuda.synchronize()
    whole = q.decodePerChannel(q.encodePerChannel(X.reshape(-1), config=cfg))
    assert np.array_equal(out.cpu().numpy(), whole)


def test_channel_append_requires_group_boundary(q):
    import pitch_amd as P
    X = offset_keys(64, 16, 2)
    a = q.encodePerChannel(X.reshape(-1), dim=16, bits=4)
    a.append(q.encodePerChannel(X[:10].reshape(-1), dim=16, bits=4))
    assert a.count == 74 and a.groupCount == 2
    with pytest.raises(P.PITCHError):
        a.append(q.encodePerChannel(X.reshape(-1), dim=16, bits=4))


def test_channel_rejects_invalid_values(q):
    import pitch_amd as P
    for x in ([1.0, 2.0, 3.0], [1.0, np.nan], [1.0, 70000.0]):
        with pytest.raises(P.PITCHError):
            q.encodePerChannel(np.array(x, np.float32), dim=2, bits=4)


@pytest.mark.parametrize("d,G", [(1, 1), (3, 7), (17, 64), (64, 16), (100, 256), (1000, 64), (1024, 33)])
@pytest.mark.parametrize("bits", [2, 3, 5, 8])
def test_channel_against_oracle(q, d, G, bits):
    import pitch_amd as P
    n = 300 if d < 512 else 70
    X = offset_keys(n, d, d + G + bits) if d >= 4 else gaussian(n, d, d + G)
    cfg = P.ChannelQuantConfig(d, bits, G)
    ours = q.encodePerChannel(X.reshape(-1), config=cfg)
    codes, ranges = O.channel_encode(X, bits, G)
    assert np.array_equal(ours.ranges, ranges.view(np.uint16).reshape(-1))
    assert ours.codes == O.pack_codes(codes, bits)
    dec = q.decodePerChannel(ours)
    ref = O.channel_decode(codes, ranges, bits, G)
    assert np.array_equal(dec.view(np.uint32), ref.reshape(-1).view(np.uint32))


# ----------------------------------------------------------------------------- function-level mirrors
@pytest.mark.parametrize("method", METHODS)
@pytest.mark.parametrize("d,bits", [(16, 3), (64, 4), (128, 2), (512, 8)])
def test_function_mirrors(q, method, d, bits):
    """pitch_amd.turbo_encode / polar_* / pack_codes / unpack_codes on device tensors (pitch_reference.py:68-132)."""
    import torch
    import pitch_amd as P
    X = gaussian(200, d, d + bits)
    x = torch.from_numpy(X).to(q.device)
    codes, scales = P.ENCODERS[method](x, bits, 0x00C0FFEE)
    ref_codes, ref_scales = O.ENCODERS[method](X.astype(np.float64), bits, 0x00C0FFEE)
    got = codes.cpu().numpy()
    check_codes(method, X, bits, 0x00C0FFEE, O.pack_codes(got, bits), O.pack_codes(ref_codes, bits), "mirror")
    check_scales(scales.cpu().numpy(), np.asarray(ref_scales, np.float32), "mirror")
    rec = P.DECODERS[method](codes, scales, bits, 0x00C0FFEE).cpu().numpy()
    ref = O.DECODERS[method](got, scales.cpu().numpy().astype(np.float64), bits, 0x00C0FFEE)
    assert max_rel_diff(rec, ref, d) < REL_L2_BAR
    packed = P.pack_codes(codes, bits)
    assert packed.cpu().numpy().tobytes() == O.pack_codes(got, bits)
    assert torch.equal(P.unpack_codes(packed, 200, d, bits), codes)


@pytest.mark.parametrize("d,bits,G", [(7, 3, 16), (64, 4, 64), (128, 8, 100)])
def test_channel_function_mirrors(q, d, bits, G):
    import torch
    import pitch_amd as P
    X = offset_keys(150, d, d) if d >= 4 else gaussian(150, d, d)
    codes, ranges = P.channel_encode(torch.from_numpy(X).to(q.device), bits, G)
    ref_codes, ref_ranges = O.channel_encode(X, bits, G)
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(ranges.cpu().numpy().view(np.uint16), ref_ranges.view(np.uint16))
    dec = P.channel_decode(codes, ranges, bits, G).cpu().numpy()
    assert np.array_equal(dec.view(np.uint32), O.channel_decode(ref_codes, ref_ranges, bits, G).view(np.uint32))
