"""The host-side operator surface without a GPU (CPU only): configs, containers, validation, accounting.

Mirrors the reference's host-side tests: BatchAPITests (constructorValidatesSizes, perVectorAccounting,
batchAccountingIncludesHeader, codable round trip and format-version checks, appendRejectsDifferentConfig;
Tests/PITCHTests/BatchAPITests.swift:32-186), PerChannelTests (rejectsInvalidArguments, storageAccounting,
halfConversion, appendRequiresGroupBoundary; Tests/PITCHTests/PerChannelTests.swift:174-221) and
CodecTests' input validation (Tests/PITCHTests/CodecTests.swift:121-150). Containers are built from synthetic
codes here; the GPU tests build them with the kernels.
"""
import json

import numpy as np
import pytest

import pitch_amd as P
from pitch_amd import api
from oracle import pitch_oracle as O


@pytest.fixture(autouse=True)
def _lib_built(built_library):
    return built_library


def _batch(cfg, n, seed=0):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, n * cfg.codeStride, dtype=np.uint8).tobytes()
    return P.CompressedBatch(cfg, codes, rng.uniform(0, 5, n).astype(np.float32))


# ----------------------------------------------------------------------------- configs
def test_per_vector_accounting():
    t = P.QuantConfig("turboQuant", 64, 3)
    assert (t.codeStride, t.bytesPerVector, t.bitsPerCoordinate) == (24, 28, 3.5)
    p = P.QuantConfig(P.QuantMethod.polarQuant, 1024, 4)
    assert p.bytesPerVector == 516
    assert abs(p.compressionRatio - 4096.0 / 516.0) < 1e-12
    kv = P.QuantConfig("turboQuant", 64, 4)
    assert abs(kv.compressionRatioVsFloat16 - 16.0 / 4.5) < 1e-12
    assert abs(kv.compressionRatio - 32.0 / 4.5) < 1e-12
    assert P.QuantConfig("turboQuant", 2, 3).codeStride == 4
    assert kv.seed == P.DEFAULT_SEED == 0x50495443


@pytest.mark.parametrize("dim", [0, 1, 3, 100, 2048])
def test_invalid_dimension(dim):
    with pytest.raises(P.InvalidDimension):
        P.QuantConfig("turboQuant", dim, 4)


@pytest.mark.parametrize("bits", [0, 1, 9, 16])
def test_invalid_bits(bits):
    with pytest.raises(P.InvalidBitWidth):
        P.QuantConfig("polarQuant", 64, bits)


def test_invalid_method_and_seed():
    with pytest.raises(P.InvalidInput):
        P.QuantConfig("kivi", 64, 4)
    with pytest.raises(P.InvalidInput):
        P.QuantConfig("turboQuant", 64, 4, 2 ** 32)
    assert issubclass(P.InvalidDimension, P.PITCHError)


def test_channel_config_validation_and_accounting():
    for args in [(0, 4), (2048, 4), (64, 1), (64, 4, 0)]:
        with pytest.raises(P.PITCHError):
            P.ChannelQuantConfig(*args)
    c = P.ChannelQuantConfig(64, 4)
    assert c.bitsPerCoordinate == 4.5
    assert P.ChannelQuantConfig(128, 4).bitsPerCoordinate == 4.5
    assert P.ChannelQuantConfig(128, 4, 128).bitsPerCoordinate == 4.25
    assert abs(c.compressionRatioVsFloat16 - 16.0 / 4.5) < 1e-12
    assert (c.codeStride, c.rangeStride, c.groupCount(150)) == (32, 256, 3)
    assert P.ChannelQuantConfig(96, 3).codeStride == 36


# ----------------------------------------------------------------------------- CompressedBatch
def test_batch_constructor_validates_sizes():
    cfg = P.QuantConfig("turboQuant", 64, 4)
    for codes, scales in [(bytes(cfg.codeStride - 4), [1]), (bytes(cfg.codeStride), [1, 2]),
                          (bytes(cfg.codeStride), [np.nan]), (bytes(0), []), (bytes(cfg.codeStride), [-1])]:
        with pytest.raises(P.InvalidInput):
            P.CompressedBatch(cfg, codes, np.array(scales, np.float32))


def test_batch_accounting_includes_header():
    b = _batch(P.QuantConfig("turboQuant", 64, 3), 100)
    assert b.payloadByteCount == 100 * 24
    assert b.sideInformationByteCount == 100 * 4 + P.CompressedBatch.headerByteCount
    assert b.storedByteCount == 2816 and b.originalByteCount == 25600
    assert abs(b.bitsPerCoordinate - 2816.0 * 8 / 6400) < 1e-12
    assert abs(b.compressionRatioVsFloat16 - 12800.0 / 2816.0) < 1e-12


def test_batch_append_and_slice_round_trip():
    whole = _batch(P.QuantConfig("polarQuant", 64, 4), 10, 3)
    built = whole.vectors(range(0, 3))
    built.append(whole.vectors(range(3, 10)))
    assert built == whole and built.count == 10
    with pytest.raises(P.InvalidInput):
        whole.vectors(range(5, 11))
    with pytest.raises(P.ConfigurationMismatch):
        built.append(_batch(P.QuantConfig("polarQuant", 64, 3), 1))


def test_batch_json_round_trip_and_version():
    b = _batch(P.QuantConfig("polarQuant", 128, 3, 99), 5, 4)
    back = P.CompressedBatch.from_json(b.to_json())
    assert back == b and back.config.seed == 99
    obj = json.loads(b.to_json())
    obj["formatVersion"] = P.CompressedBatch.formatVersion + 1
    with pytest.raises(P.InvalidInput):
        P.CompressedBatch.from_json(json.dumps(obj))
    bad = '{"formatVersion":3,"config":{"method":"turboQuant","dim":100,"bits":4,"seed":1},"codes":"","scales":[1]}'
    with pytest.raises(P.PITCHError):
        P.CompressedBatch.from_json(bad)


def _swift_base64(data: bytes) -> str:
    """Base64 as Swift's JSONEncoder writes Data (.base64), with '/' escaped as '\\/' (its default)."""
    import base64
    return base64.b64encode(data).decode().replace("/", "\\/")


def test_batch_json_as_swift_writes_it():
    """A CompressedBatch document laid out by the reference's CodingKeys (CompressedBatch.swift:95-121:
    formatVersion, config, codes, scales; QuantConfig.swift:37: method, dim, bits, seed), written the way Swift's
    JSONEncoder does (Data as base64 with escaped slashes, [Float] as shortest round-trip numbers, keys in any
    order, compact or pretty-printed), parses to the same batch; malformed documents raise InvalidInput."""
    codes = bytes([0xFB, 0xFF, 0xBF, 0x00, 0x01, 0x02, 0x03, 0xFE, 0x3F, 0x10, 0x20, 0x30])
    b64 = _swift_base64(codes)
    assert "\\/" in b64
    compact = ('{"scales":[1.5,0.1,3.1415927],"formatVersion":3,"codes":"%s","config":{"seed":1346982979,"bits":4,'
               '"method":"turboQuant","dim":8}}' % b64)
    pretty = ('{\n  "codes" : "%s",\n  "config" : {\n    "bits" : 4,\n    "dim" : 8,\n    "method" : "turboQuant",\n'
              '    "seed" : 1346982979\n  },\n  "formatVersion" : 3,\n  "scales" : [\n    1.5,\n    0.1,\n'
              '    3.1415927\n  ]\n}' % b64)
    for doc in (compact, pretty):
        b = P.CompressedBatch.from_json(doc)
        assert b.codes == codes and b.count == 3
        assert (b.config.method, b.config.dim, b.config.bits, b.config.seed) == ("turboQuant", 8, 4, 0x50495443)
        assert np.array_equal(b.scales, np.array([1.5, 0.1, 3.1415927], np.float32))
        assert P.CompressedBatch.from_json(b.to_json()) == b
    bad = [compact.replace('"formatVersion":3', '"formatVersion":2'),       # other version
           compact.replace(b64, "@@@@" + b64[4:]),                          # not base64
           compact.replace('"scales":[1.5,0.1,3.1415927],', ""),            # missing key
           compact.replace("1.5,", '"1.5",'),                               # wrong element type
           compact.replace('"turboQuant"', '"fooQuant"'),                   # unknown method
           compact.replace('[1.5,0.1,3.1415927]', '[1.5,0.1]'),             # scales do not match the codes
           "[]", "not json"]
    for doc in bad:
        with pytest.raises(P.InvalidInput):
            P.CompressedBatch.from_json(doc)
    with pytest.raises(P.InvalidDimension):
        P.CompressedBatch.from_json(compact.replace('"dim":8', '"dim":12'))


def test_block_json_as_swift_writes_it():
    """A ChannelCompressedBlock document laid out by the reference's CodingKeys (PerChannel.swift:143-168:
    formatVersion, config, codes, ranges; :45: dim, bits, groupSize; ranges as [UInt16]), as Swift's JSONEncoder
    writes it, parses to the same block, including a partial last group and a negative-zero minimum."""
    codes = bytes(range(0xF0, 0xFC))                        # 3 tokens x codeStride 4
    ranges = [0xBC00, 0x0000, 0x3C00, 0x3C00, 0x4000, 0x4000,  # group 0: min row, max row
              0x8000, 0x3800, 0xC000, 0x0000, 0x3C00, 0x0000]  # group 1 (one token): -0.0 .. 0.0, 0.5 .. 1, -2 .. 0
    doc = ('{"ranges":[%s],"formatVersion":1,"config":{"groupSize":2,"dim":3,"bits":4},"codes":"%s"}'
           % (",".join(str(r) for r in ranges), _swift_base64(codes)))
    blk = P.ChannelCompressedBlock.from_json(doc)
    assert blk.codes == codes and blk.count == 3 and blk.groupCount == 2
    assert (blk.config.dim, blk.config.bits, blk.config.groupSize) == (3, 4, 2)
    assert blk.ranges.dtype == np.uint16 and blk.ranges.tolist() == ranges
    assert blk.range(1, 0) == (-0.0, 0.0) and np.signbit(blk.range(1, 0)[0])
    assert P.ChannelCompressedBlock.from_json(blk.to_json()) == blk
    for bad in (doc.replace('"formatVersion":1', '"formatVersion":3'), doc.replace("48128", "70000"),
                doc.replace("48128", "-1"), doc.replace('"groupSize":2', '"groupSize":0'),
                doc.replace("15360,15360", "15360")):
        with pytest.raises(P.InvalidInput):
            P.ChannelCompressedBlock.from_json(bad)


# ----------------------------------------------------------------------------- ChannelCompressedBlock
def _block(cfg, n, seed=0):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, cfg.dim)).astype(np.float32)
    codes, ranges = O.channel_encode(X, cfg.bits, cfg.groupSize)
    return P.ChannelCompressedBlock(cfg, O.pack_codes(codes, cfg.bits), ranges.view(np.uint16).reshape(-1))


def test_block_validation():
    cfg = P.ChannelQuantConfig(4, 4)
    with pytest.raises(P.InvalidInput):                                    # ranges too short
        P.ChannelCompressedBlock(cfg, bytes(4), np.array([0, 0], np.uint16))
    with pytest.raises(P.InvalidInput):                                    # min above max (2.0 > 1.0)
        P.ChannelCompressedBlock(cfg, bytes(4), np.array([0x4000, 0, 0, 0, 0x3C00, 0, 0, 0], np.uint16))
    with pytest.raises(P.InvalidInput):                                    # infinite range
        P.ChannelCompressedBlock(cfg, bytes(4), np.array([0, 0, 0, 0, 0x7C00, 0, 0, 0], np.uint16))
    with pytest.raises(P.InvalidInput):
        P.ChannelCompressedBlock(cfg, bytes(3), np.zeros(8, np.uint16))
    ok = P.ChannelCompressedBlock(cfg, bytes(4), np.array([0, 0, 0, 0, 0x3C00, 0, 0, 0], np.uint16))
    assert ok.range(0, 0) == (0.0, 1.0)


def test_block_append_requires_group_boundary():
    cfg = P.ChannelQuantConfig(16, 4)
    a = _block(cfg, 64, 1)
    a.append(_block(cfg, 10, 2))
    assert a.count == 74 and a.groupCount == 2
    with pytest.raises(P.InvalidInput):
        a.append(_block(cfg, 64, 3))
    with pytest.raises(P.ConfigurationMismatch):
        _block(cfg, 64).append(_block(P.ChannelQuantConfig(16, 3), 64))


def test_block_storage_accounting_and_json():
    c = P.ChannelQuantConfig(64, 4)
    block = _block(c, 128, 5)
    assert block.storedByteCount == 128 * 32 + 2 * 256 + P.ChannelCompressedBlock.headerByteCount
    assert block.groupCount == 2
    b2 = _block(P.ChannelQuantConfig(32, 3, 32), 70, 4)
    assert P.ChannelCompressedBlock.from_json(b2.to_json()) == b2
    obj = json.loads(b2.to_json())
    obj["formatVersion"] = 2
    with pytest.raises(P.InvalidInput):
        P.ChannelCompressedBlock.from_json(json.dumps(obj))


def test_half_conversion():
    """PerChannelTests.halfConversion (PerChannelTests.swift:214-221)."""
    assert P.half_to_float(0x3C00) == 1.0
    assert P.half_to_float(0xC000) == -2.0
    assert P.half_to_float(0x7BFF) == 65504.0
    assert P.half_to_float(0x0001) == 2.0 ** -24
    assert P.half_to_float(0x7C00) == float("inf")
    assert np.isnan(P.half_to_float(0x7E00))


# ----------------------------------------------------------------------------- value validation
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf, 1e30, -1e18])
@pytest.mark.parametrize("pos", [0, 37, 4095])
def test_invalid_values(bad, pos):
    """CodecTests.invalidValuesThrow (CodecTests.swift:145-149)."""
    x = np.full(4096, 0.5, np.float32)
    x[pos] = bad
    with pytest.raises(P.InvalidInput):
        api._validate_values(x, P.QuantConfig.maxInputMagnitude, "")


def test_value_limits():
    api._validate_values(np.full(1024, 1e17, np.float32), P.QuantConfig.maxInputMagnitude, "")
    api._validate_values(np.array([65504.0], np.float32), P.ChannelQuantConfig.maxInputMagnitude, "")
    with pytest.raises(P.InvalidInput):
        api._validate_values(np.array([1.0, 70000.0], np.float32), P.ChannelQuantConfig.maxInputMagnitude, "")


# ----------------------------------------------------------------------------- host mirrors
def test_function_mirrors_match_oracle():
    for d in O.SUPPORTED_DIMS:
        for b in O.SUPPORTED_BITS:
            assert P.code_stride_bytes(d, b) == O.code_stride_bytes(d, b)
            assert P.bits_per_coordinate(d, b) == O.bits_per_coordinate(d, b)
        assert np.array_equal(P.rand_signs(0x00C0FFEE, d), O.rand_signs(0x00C0FFEE, d))
    assert P.channel_bits_per_coordinate(96, 3, 16) == O.channel_bits_per_coordinate(96, 3, 16)


def test_no_device_raises_loudly():
    """Without a GPU the codec refuses to run; there is no CPU fallback."""
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(P.DeviceUnavailable):
        P.PITCH()


def test_product_never_imports_the_oracle():
    import pathlib
    pkg = pathlib.Path(P.__file__).resolve().parent
    for f in list(pkg.rglob("*.py")):
        text = f.read_text()
        assert "oracle" not in text, f"{f} mentions the oracle"
