"""GPU parity of the float16 / bfloat16 entry points (pitch_enqueue_*_io).

They are specified as the conversion the reference leaves to its callers ("Inputs and outputs are float32;
models that keep caches in fp16 or bf16 need a conversion", README.md:97):
* encoding 16-bit vectors gives the same codes, scales and ranges, byte for byte, as encoding their exact
  float32 widening through the float32 entry point, and so meets the oracle on those float32 values to the
  usual bar (per-vector codes outside the near-boundary band and KIVI codes and ranges bit-exact);
* decoding to a 16-bit type gives the float32 decode rounded to nearest even: bit-exact against the oracle's
  rounding (tests/test_io_rounding.py pins it) of the library's own float32 decode, bit-exact against the
  oracle's KIVI decode rounded the same way, and for the per-vector methods within 1e-5 plus the type's
  half-ulp (2^-11 for float16, 2^-8 for bfloat16) relative L2 per vector of the oracle's float32 decode;
* slices at byte offsets into 16-bit caches give the same bytes as whole calls.
Every call goes through libpitch_amd.so's C ABI.
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O
from test_gpu_parity import REL_L2_BAR, check_codes, max_rel_diff

pytestmark = pytest.mark.gpu

IO_DTYPES = ["float16", "bfloat16"]
HALF_ULP = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}   # relative rounding error of a 16-bit store


def _tdtype(io):
    import torch
    return getattr(torch, io)


def _bits16(t):
    """Bit patterns of a 16-bit device tensor as uint16 numpy."""
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _inputs(n, d, seed, dev, io):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(n, d, generator=g, device=dev)
    x *= torch.exp(torch.empty(n, 1, device=dev).uniform_(-3, 3, generator=g))
    return x.to(_tdtype(io)).contiguous()


PER_VECTOR = [(m, d, b) for m in ("turboQuant", "polarQuant") for d in (2, 8, 64, 128, 256, 1024) for b in (2, 4, 8)]


@pytest.mark.parametrize("io", IO_DTYPES)
@pytest.mark.parametrize("method,d,bits", PER_VECTOR)
def test_per_vector_encode_16bit(q, method, d, bits, io):
    import torch
    import pitch_amd as P
    n = 777 if d <= 256 else 203
    print(f"encode {io} {method} d={d} b={bits} n={n}", flush=True)
    cfg = P.QuantConfig(method, d, bits)
    x16 = _inputs(n, d, 100 * d + bits, q.device, io)
    x32 = x16.float().contiguous()
    c16 = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    s16 = torch.empty(n, dtype=torch.float32, device=q.device)
    c32, s32 = torch.empty_like(c16), torch.empty_like(s16)
    q.enqueueEncode(x16, c16, s16, n, cfg)
    q.enqueueEncode(x32, c32, s32, n, cfg)
    torch.cuda.synchronize()
    assert torch.equal(c16, c32) and torch.equal(s16, s32)
    X = x32.cpu().numpy()
    ref_codes, ref_scales = O.ENCODERS[method](X.astype(np.float64), bits)
    check_codes(method, X, bits, P.DEFAULT_SEED, c16.cpu().numpy().tobytes(), O.pack_codes(ref_codes, bits),
                f"{io} {method} d={d} b={bits}")
    ulps = np.abs(s16.cpu().numpy().view(np.int32).astype(np.int64)
                  - np.asarray(ref_scales, np.float32).view(np.int32).astype(np.int64))
    assert ulps.max() <= 1


@pytest.mark.parametrize("io", IO_DTYPES)
@pytest.mark.parametrize("method,d,bits,n", [("polarQuant", 64, 3, 777), ("polarQuant", 64, 5, 1000),
                                             ("turboQuant", 128, 3, 1000), ("polarQuant", 128, 5, 777),
                                             ("polarQuant", 128, 5, (3 << 20) + 45), ("turboQuant", 128, 3, (3 << 20) + 45)])
def test_staged_encoder_16bit_odd_bits_and_long_calls(q, method, d, bits, n, io):
    """16-bit vectors through the staged-stage encoder (PolarQuant at d = 64 / 128, TurboQuant at d = 128): odd bit
    widths (code words shared between lanes at d = 64) and calls of more than 56 resident rounds (the grid of about
    8 blocks per workgroup) give the bytes of the float32 encode of the widened values, which the float32 parity
    tests pin against the oracle."""
    import torch
    import pitch_amd as P
    print(f"staged 16-bit {io} {method} d={d} b={bits} n={n}", flush=True)
    cfg = P.QuantConfig(method, d, bits)
    x16 = _inputs(n, d, 31 * d + bits, q.device, io)
    x32 = x16.float().contiguous()
    c16 = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    s16 = torch.empty(n, dtype=torch.float32, device=q.device)
    c32, s32 = torch.empty_like(c16), torch.empty_like(s16)
    q.enqueueEncode(x16, c16, s16, n, cfg)
    q.enqueueEncode(x32, c32, s32, n, cfg)
    torch.cuda.synchronize()
    assert torch.equal(c16, c32) and torch.equal(s16.view(torch.int32), s32.view(torch.int32))
    del x16, x32, c16, s16, c32, s32
    torch.cuda.empty_cache()


@pytest.mark.parametrize("io", IO_DTYPES)
@pytest.mark.parametrize("method,d,bits", PER_VECTOR)
def test_per_vector_decode_16bit(q, method, d, bits, io):
    import torch
    import pitch_amd as P
    n = 777 if d <= 256 else 203
    print(f"decode {io} {method} d={d} b={bits} n={n}", flush=True)
    cfg = P.QuantConfig(method, d, bits)
    rng = np.random.default_rng(7 * d + bits)
    codes = rng.integers(0, 2 ** bits, (n, d))
    scales = np.exp(rng.uniform(-4, 4, n)).astype(np.float32)
    packed = torch.from_numpy(np.frombuffer(O.pack_codes(codes, bits), np.uint8).copy()).to(q.device)
    sc = torch.from_numpy(scales).to(q.device)
    o32 = torch.empty(n, d, dtype=torch.float32, device=q.device)
    o16 = torch.empty(n, d, dtype=_tdtype(io), device=q.device)
    q.enqueueDecode(packed, sc, o32, n, cfg)
    q.enqueueDecode(packed, sc, o16, n, cfg)
    torch.cuda.synchronize()
    ours = _bits16(o16)
    assert np.array_equal(ours, O.to_io_bits(o32.cpu().numpy(), io).reshape(n, d))
    ref = O.DECODERS[method](codes, scales.astype(np.float64), bits)
    assert max_rel_diff(O.from_io_bits(ours, io), ref, d) < REL_L2_BAR + HALF_ULP[io]


CHANNEL = [(64, 64, 4), (128, 64, 2), (12, 7, 3), (128, 100, 8), (64, 128, 4), (33, 64, 5), (1024, 64, 4),
           # eight channels per lane in the wave decoder: b = 3 rows straddle code words; d = 96 keeps four
           (128, 64, 3), (192, 128, 2), (96, 64, 4)]


@pytest.mark.parametrize("io", IO_DTYPES)
@pytest.mark.parametrize("d,G,bits", CHANNEL)
def test_channel_16bit(q, d, G, bits, io):
    """Covers every per-channel kernel: the wave encoder (d % 4 = 0, G <= 64), the two-pass encoder (G > 64),
    the per-element encoder (d % 4 != 0), and the wave, vec4 and per-element decoders."""
    import torch
    import pitch_amd as P
    n = 3 * G + G // 2 + 1
    print(f"KIVI {io} d={d} G={G} b={bits} n={n}", flush=True)
    cfg = P.ChannelQuantConfig(d, bits, G)
    groups = cfg.groupCount(n)
    g = torch.Generator(device=q.device)
    g.manual_seed(d * G + bits)
    x = torch.randn(n, d, generator=g, device=q.device) * torch.exp(torch.randn(d, generator=g, device=q.device))
    x += 3 * torch.randn(d, generator=g, device=q.device)
    x16 = x.to(_tdtype(io)).contiguous()
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    ranges = torch.empty(groups * 2 * d, dtype=torch.float16, device=q.device)
    codes32, ranges32 = torch.empty_like(codes), torch.empty_like(ranges)
    q.enqueuePerChannelEncode(x16, codes, ranges, n, cfg)
    q.enqueuePerChannelEncode(x16.float().contiguous(), codes32, ranges32, n, cfg)
    out16 = torch.empty(n, d, dtype=_tdtype(io), device=q.device)
    q.enqueuePerChannelDecode(codes, ranges, out16, n, cfg)
    torch.cuda.synchronize()
    assert torch.equal(codes, codes32) and torch.equal(ranges, ranges32)
    X = x16.float().cpu().numpy()
    ref_codes, ref_ranges = O.channel_encode(X, bits, G)
    assert codes.cpu().numpy().tobytes() == O.pack_codes(ref_codes, bits)
    assert np.array_equal(ranges.cpu().numpy().view(np.uint16), ref_ranges.view(np.uint16).reshape(-1))
    ref = O.channel_decode(ref_codes, ref_ranges, bits, G)
    assert np.array_equal(_bits16(out16), O.to_io_bits(ref, io).reshape(n, d))


@pytest.mark.parametrize("io", IO_DTYPES)
def test_16bit_slices_at_byte_offsets(q, io):
    """A slice encoded or decoded through byte offsets into 16-bit caches equals the same bytes of one whole
    call (offsets in bytes, multiples of 4, as for float32)."""
    import torch
    import pitch_amd as P
    n, d, lo, m = 5000, 128, 1234, 777
    cfg = P.QuantConfig("turboQuant", d, 3)
    x16 = _inputs(n, d, 9, q.device, io)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    scales = torch.empty(n, dtype=torch.float32, device=q.device)
    q.enqueueEncode(x16, codes, scales, n, cfg)
    c2 = torch.zeros(m * cfg.codeStride, dtype=torch.uint8, device=q.device)
    s2 = torch.zeros(m, dtype=torch.float32, device=q.device)
    q.enqueueEncode(x16, c2, s2, m, cfg, inputOffset=lo * d * 2)
    whole = torch.empty(n, d, dtype=_tdtype(io), device=q.device)
    q.enqueueDecode(codes, scales, whole, n, cfg)
    part = torch.zeros(n, d, dtype=_tdtype(io), device=q.device)
    q.enqueueDecode(codes, scales, part, m, cfg, codesOffset=lo * cfg.codeStride, scalesOffset=lo * 4,
                    outputOffset=lo * d * 2)
    torch.cuda.synchronize()
    assert torch.equal(c2, codes[lo * cfg.codeStride:(lo + m) * cfg.codeStride])
    assert torch.equal(s2, scales[lo:lo + m])
    assert torch.equal(part[lo:lo + m].view(torch.int16), whole[lo:lo + m].view(torch.int16))
    assert not part[:lo].view(torch.int16).any() and not part[lo + m:].view(torch.int16).any()
    # per-channel: one head of a two-head 16-bit cache, at its offsets
    kc = P.ChannelQuantConfig(64, 4, 64)
    T = 640
    keys = _inputs(2 * T, 64, 11, q.device, io)
    kcodes = torch.empty(2 * T * kc.codeStride, dtype=torch.uint8, device=q.device)
    kr = torch.empty(2 * kc.groupCount(T) * 2 * 64, dtype=torch.float16, device=q.device)
    q.enqueuePerChannelEncode(keys, kcodes, kr, T, kc, inputOffset=T * 64 * 2, codesOffset=T * kc.codeStride,
                              rangesOffset=kc.groupCount(T) * kc.rangeStride)
    kout = torch.zeros(2 * T, 64, dtype=_tdtype(io), device=q.device)
    q.enqueuePerChannelDecode(kcodes, kr, kout, T, kc, codesOffset=T * kc.codeStride,
                              rangesOffset=kc.groupCount(T) * kc.rangeStride, outputOffset=T * 64 * 2)
    torch.cuda.synchronize()
    X = keys[T:].float().cpu().numpy()
    ref_codes, ref_ranges = O.channel_encode(X, 4, 64)
    assert kcodes[T * kc.codeStride:].cpu().numpy().tobytes() == O.pack_codes(ref_codes, 4)
    ref = O.channel_decode(ref_codes, ref_ranges, 4, 64)
    assert np.array_equal(_bits16(kout[T:]), O.to_io_bits(ref, io).reshape(T, 64))
    assert not kout[:T].view(torch.int16).any()


def test_function_mirrors_keep_16bit(q):
    """turbo_encode / channel_encode read 16-bit tensors directly; dtype= selects a 16-bit decode."""
    import torch
    import pitch_amd as P
    x = _inputs(300, 64, 3, q.device, "bfloat16")
    codes, norms = P.turbo_encode(x, 4)
    codes32, norms32 = P.turbo_encode(x.float(), 4)
    assert torch.equal(codes, codes32) and torch.equal(norms, norms32)
    out = P.turbo_decode(codes, norms, 4, dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    ref = P.turbo_decode(codes, norms, 4)
    assert np.array_equal(_bits16(out), O.to_io_bits(ref.cpu().numpy(), "bfloat16").reshape(300, 64))
    kc, kr = P.channel_encode(x.to(torch.float16), 4)
    dec = P.channel_decode(kc, kr, 4, dtype=torch.float16)
    assert dec.dtype == torch.float16


@pytest.mark.parametrize("io", IO_DTYPES)
@pytest.mark.parametrize("d,bits", [(64, 4), (128, 3), (192, 2)])
def test_channel_16bit_long_decode(q, d, bits, io):
    """A 16-bit per-channel decode of several launches' worth of tokens (partial last group; long enough for the
    wave decoder's eight channels per lane) equals the float32 decode of the same codes rounded to the 16-bit
    type, bit for bit (torch's casts round to nearest even, as
    the oracle's 16-bit rules do)."""
    import torch
    import pitch_amd as P
    n, G = (1 << 20) + 37, 64
    print(f"KIVI long decode {io} d={d} b={bits} n={n}", flush=True)
    cfg = P.ChannelQuantConfig(d, bits, G)
    g = torch.Generator(device=q.device)
    g.manual_seed(n + d + bits)
    x = torch.randn(n, d, generator=g, device=q.device) * 4
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    ranges = torch.empty(cfg.groupCount(n) * 2 * d, dtype=torch.float16, device=q.device)
    q.enqueuePerChannelEncode(x, codes, ranges, n, cfg)
    out32 = torch.empty(n, d, dtype=torch.float32, device=q.device)
    out16 = torch.empty(n, d, dtype=_tdtype(io), device=q.device)
    q.enqueuePerChannelDecode(codes, ranges, out32, n, cfg)
    q.enqueuePerChannelDecode(codes, ranges, out16, n, cfg)
    torch.cuda.synchronize()
    assert torch.equal(out16.view(torch.int16), out32.to(_tdtype(io)).view(torch.int16))
