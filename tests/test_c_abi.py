"""The C ABI of libpitch_amd.so without a GPU (CPU only): exports, configs and argument validation.

Every symbol declared in include/pitch_amd.h must be exported and bound by pitch_amd/_lib.py. The config
entry points and the enqueue entry points' argument checks need no device: they mirror QuantConfig.init
(Sources/PITCH/Models/QuantConfig.swift:24-40), ChannelQuantConfig.init (Sources/PITCH/PerChannel.swift:36-52)
and the buffer checks of Sources/PITCH/Core/Codec.swift:30-47 and PerChannel.swift:318-374, and they all run
before the library looks for a device. The buffers passed here are host memory and never reach a kernel:
every call either fails validation or stops at the device-memory check.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from pitch_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "pitch_amd.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pitch_[a-z0-9_]+)\s*\(", text)))


def header_defines():
    return {m.group(1): int(m.group(2)) for m in
            re.finditer(r"#define\s+(PITCH_(?:OK|ERR_[A-Z_]+))\s+\(?(-?\d+)\)?", HEADER.read_text())}


@pytest.fixture(scope="module")
def lib(built_library):
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = header_functions()
    assert len(names) >= 10
    assert set(names) == set(_lib.SIGNATURES), "header and ctypes binding disagree"
    for n in names:
        assert hasattr(lib, n), f"{n} not exported"
    dyn = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True)
    if dyn.returncode == 0:
        exported = {line.split()[-1] for line in dyn.stdout.splitlines() if line.strip()}
        assert set(names) <= exported


def test_error_codes_match_header():
    d = header_defines()
    assert d["PITCH_OK"] == _lib.PITCH_OK == 0
    assert d["PITCH_ERR_INVALID_INPUT"] == _lib.ERR_INVALID_INPUT
    assert d["PITCH_ERR_INVALID_BIT_WIDTH"] == _lib.ERR_INVALID_BIT_WIDTH
    assert d["PITCH_ERR_INVALID_DIMENSION"] == _lib.ERR_INVALID_DIMENSION
    assert d["PITCH_ERR_CONFIGURATION_MISMATCH"] == _lib.ERR_CONFIGURATION_MISMATCH
    assert d["PITCH_ERR_ENCODING_FAILED"] == _lib.ERR_ENCODING_FAILED
    assert d["PITCH_ERR_DECODING_FAILED"] == _lib.ERR_DECODING_FAILED
    assert d["PITCH_ERR_DEVICE_UNAVAILABLE"] == _lib.ERR_DEVICE_UNAVAILABLE


def test_version(lib):
    assert lib.pitch_version() == 0x000200


def _config(lib, method, dim, bits, seed=0x50495443):
    c = _lib.PitchConfigC()
    cs = ctypes.c_uint32(0)
    rc = lib.pitch_config(method, dim, bits, seed, ctypes.byref(c), ctypes.byref(cs))
    return rc, c, cs.value


def test_config_all_valid(lib):
    for method in (0, 1):
        for dim in [2 ** k for k in range(1, 11)]:
            for bits in range(2, 9):
                rc, c, cs = _config(lib, method, dim, bits, 7)
                assert rc == 0
                assert (c.method, c.dim, c.bits, c.seed) == (method, dim, bits, 7)
                assert cs == ((dim * bits + 7) // 8 + 3) & ~3        # reference/pitch_reference.py:65-66


@pytest.mark.parametrize("dim", [0, 1, 3, 100, 2048, 4096])
def test_config_invalid_dimension(lib, dim):
    """CodecTests.invalidDimensionThrows (Tests/PITCHTests/CodecTests.swift:121-126)."""
    rc, _, _ = _config(lib, 0, dim, 4)
    assert rc == _lib.ERR_INVALID_DIMENSION
    assert "dimension" in _lib.last_error().lower()


@pytest.mark.parametrize("bits", [0, 1, 9, 16])
def test_config_invalid_bits(lib, bits):
    """CodecTests.invalidBitWidthThrows (CodecTests.swift:128-133)."""
    rc, _, _ = _config(lib, 1, 64, bits)
    assert rc == _lib.ERR_INVALID_BIT_WIDTH
    assert "bit width" in _lib.last_error().lower()


def test_config_invalid_method_and_null_outputs(lib):
    assert _config(lib, 2, 64, 4)[0] == _lib.ERR_INVALID_INPUT
    assert lib.pitch_config(0, 64, 4, 0, None, None) == 0


def _channel_config(lib, dim, bits, G):
    c = _lib.PitchChannelConfigC()
    cs, rs = ctypes.c_uint32(0), ctypes.c_uint32(0)
    rc = lib.pitch_channel_config(dim, bits, G, ctypes.byref(c), ctypes.byref(cs), ctypes.byref(rs))
    return rc, c, cs.value, rs.value


def test_channel_config(lib):
    rc, c, cs, rs = _channel_config(lib, 96, 4, 64)
    assert rc == 0 and (c.dim, c.bits, c.group_size, c.reserved) == (96, 4, 64, 0)
    assert cs == 48 and rs == 384
    assert _channel_config(lib, 1, 2, 1)[0] == 0
    assert _channel_config(lib, 1024, 8, 65536)[0] == 0
    # PerChannelTests.rejectsInvalidArguments (Tests/PITCHTests/PerChannelTests.swift:186-191)
    assert _channel_config(lib, 0, 4, 64)[0] == _lib.ERR_INVALID_INPUT
    assert _channel_config(lib, 2048, 4, 64)[0] == _lib.ERR_INVALID_INPUT
    assert _channel_config(lib, 64, 1, 64)[0] == _lib.ERR_INVALID_BIT_WIDTH
    assert _channel_config(lib, 64, 4, 0)[0] == _lib.ERR_INVALID_INPUT
    assert _channel_config(lib, 64, 4, 65537)[0] == _lib.ERR_INVALID_INPUT


# ----------------------------------------------------------------------------- enqueue validation
class Host:
    """A host buffer used only as a pointer for argument checks; it never reaches a kernel."""

    def __init__(self, nbytes):
        self.buf = ctypes.create_string_buffer(max(nbytes, 1))
        self.nbytes = nbytes

    @property
    def p(self):
        return ctypes.cast(self.buf, ctypes.c_void_p)


def _enc(lib, cfg, count, inp, codes, scales, offs=(0, 0, 0)):
    return lib.pitch_enqueue_encode(ctypes.byref(cfg) if cfg is not None else None, inp.p, inp.nbytes, offs[0],
                                    codes.p, codes.nbytes, offs[1], scales.p, scales.nbytes, offs[2], count, None)


def _dec(lib, cfg, count, codes, scales, out, offs=(0, 0, 0)):
    return lib.pitch_enqueue_decode(ctypes.byref(cfg) if cfg is not None else None, codes.p, codes.nbytes, offs[0],
                                    scales.p, scales.nbytes, offs[1], out.p, out.nbytes, offs[2], count, None)


def test_enqueue_rejects_undersized_buffers(lib):
    """BatchAPITests.enqueueRejectsUndersizedBuffers (Tests/PITCHTests/BatchAPITests.swift:93-103)."""
    cfg = _lib.PitchConfigC(0, 64, 4, 0)
    rc = _enc(lib, cfg, 4, Host(64 * 4 * 4), Host(32 * 3), Host(16))      # codes need 4 * 32 bytes
    assert rc == _lib.ERR_INVALID_INPUT
    assert "codes" in _lib.last_error()
    assert _enc(lib, cfg, 4, Host(64 * 4 * 4 - 4), Host(128), Host(16)) == _lib.ERR_INVALID_INPUT
    assert _enc(lib, cfg, 4, Host(1024), Host(128), Host(12)) == _lib.ERR_INVALID_INPUT
    assert _dec(lib, cfg, 4, Host(128), Host(16), Host(1020)) == _lib.ERR_INVALID_INPUT
    # the size check counts the bytes after the offset
    assert _enc(lib, cfg, 4, Host(1024), Host(128 + 4), Host(16), offs=(0, 8, 0)) == _lib.ERR_INVALID_INPUT
    assert _enc(lib, cfg, 1, Host(1024), Host(128), Host(16), offs=(0, 256, 0)) == _lib.ERR_INVALID_INPUT


def test_enqueue_rejects_misaligned_offsets(lib):
    """BatchAPITests.enqueueRejectsMisalignedOffset (BatchAPITests.swift:105-116)."""
    cfg = _lib.PitchConfigC(1, 64, 4, 0)
    rc = _dec(lib, cfg, 1, Host(1024), Host(64), Host(4096), offs=(2, 0, 0))
    assert rc == _lib.ERR_INVALID_INPUT and "multiple of 4" in _lib.last_error()
    assert _dec(lib, cfg, 1, Host(1024), Host(64), Host(4096), offs=(0, 1, 0)) == _lib.ERR_INVALID_INPUT
    assert _enc(lib, cfg, 1, Host(1024), Host(64), Host(64), offs=(6, 0, 0)) == _lib.ERR_INVALID_INPUT


def test_enqueue_rejects_bad_config_and_count(lib):
    big = Host(1 << 16)
    assert _enc(lib, None, 1, big, big, big) == _lib.ERR_INVALID_INPUT
    assert _enc(lib, _lib.PitchConfigC(0, 100, 4, 0), 1, big, big, big) == _lib.ERR_INVALID_DIMENSION
    assert _dec(lib, _lib.PitchConfigC(0, 64, 9, 0), 1, big, big, big) == _lib.ERR_INVALID_BIT_WIDTH
    assert _dec(lib, _lib.PitchConfigC(5, 64, 4, 0), 1, big, big, big) == _lib.ERR_INVALID_INPUT
    assert _enc(lib, _lib.PitchConfigC(0, 64, 4, 0), 0, big, big, big) == _lib.ERR_INVALID_INPUT
    assert _enc(lib, _lib.PitchConfigC(0, 1024, 4, 0), 2 ** 62, big, big, big) == _lib.ERR_INVALID_INPUT
    null = Host(0)
    null.buf = None
    assert lib.pitch_enqueue_encode(ctypes.byref(_lib.PitchConfigC(0, 64, 4, 0)), None, 1 << 20, 0, big.p,
                                    big.nbytes, 0, big.p, big.nbytes, 0, 1, None) == _lib.ERR_INVALID_INPUT


def test_channel_enqueue_validation(lib):
    """PerChannel.swift:318-374: ranges need groups * 4 * dim bytes after the offset."""
    cfg = _lib.PitchChannelConfigC(64, 4, 64, 0)
    n = 150                                           # 3 groups, the last one partial
    inp, codes, ranges, out = Host(n * 256), Host(n * 32), Host(3 * 256), Host(n * 256)

    def enc(r, offs=(0, 0, 0), count=n, c=cfg):
        return lib.pitch_enqueue_channel_encode(ctypes.byref(c), inp.p, inp.nbytes, offs[0], codes.p,
                                                codes.nbytes, offs[1], r.p, r.nbytes, offs[2], count, None)

    def dec(r, offs=(0, 0, 0), count=n, c=cfg):
        return lib.pitch_enqueue_channel_decode(ctypes.byref(c), codes.p, codes.nbytes, offs[0], r.p, r.nbytes,
                                                offs[1], out.p, out.nbytes, offs[2], count, None)

    assert enc(Host(2 * 256)) == _lib.ERR_INVALID_INPUT and "ranges" in _lib.last_error()
    assert dec(Host(3 * 256 - 4)) == _lib.ERR_INVALID_INPUT
    assert enc(ranges, offs=(0, 0, 2)) == _lib.ERR_INVALID_INPUT
    assert enc(ranges, count=0) == _lib.ERR_INVALID_INPUT
    assert enc(ranges, count=2 ** 32) == _lib.ERR_INVALID_INPUT
    assert enc(ranges, c=_lib.PitchChannelConfigC(64, 4, 0, 0)) == _lib.ERR_INVALID_INPUT
    assert dec(ranges, c=_lib.PitchChannelConfigC(64, 1, 64, 0)) == _lib.ERR_INVALID_BIT_WIDTH


def test_valid_arguments_on_host_memory_stop_before_any_kernel(lib):
    """With correct sizes, host pointers are refused by the device-memory check (or, with no GPU at all,
    by the device lookup): either way an error, never a launch."""
    cfg = _lib.PitchConfigC(0, 64, 4, 0)
    rc = _enc(lib, cfg, 4, Host(1024), Host(128), Host(16))
    assert rc in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
    assert _lib.last_error()


def test_pack_entry_validation(lib):
    big = Host(1 << 12)
    assert lib.pitch_enqueue_pack_codes(0, 4, big.p, big.nbytes, 0, big.p, big.nbytes, 0, 1, None) \
        == _lib.ERR_INVALID_DIMENSION
    assert lib.pitch_enqueue_unpack_codes(64, 1, big.p, big.nbytes, 0, big.p, big.nbytes, 0, 1, None) \
        == _lib.ERR_INVALID_BIT_WIDTH
    assert lib.pitch_enqueue_pack_codes(64, 4, big.p, big.nbytes, 0, big.p, big.nbytes, 0, 0, None) \
        == _lib.ERR_INVALID_INPUT
    assert lib.pitch_enqueue_pack_codes(64, 4, big.p, 63, 0, big.p, big.nbytes, 0, 1, None) \
        == _lib.ERR_INVALID_INPUT


# ----------------------------------------------------------------------------- element-type entry points
def test_io_entry_points_validate_type_and_sizes(lib):
    """The *_io entry points size the uncompressed buffer by the element type and reject unknown types before
    looking for a device."""
    cfg = _lib.PitchConfigC(0, 64, 4, 0)
    codes, scales = Host(4 * 32), Host(16)

    def enc(io, inp):
        return lib.pitch_enqueue_encode_io(ctypes.byref(cfg), io, inp.p, inp.nbytes, 0, codes.p, codes.nbytes, 0,
                                           scales.p, scales.nbytes, 0, 4, None)

    def dec(io, out):
        return lib.pitch_enqueue_decode_io(ctypes.byref(cfg), io, codes.p, codes.nbytes, 0, scales.p,
                                           scales.nbytes, 0, out.p, out.nbytes, 0, 4, None)

    assert enc(3, Host(1024)) == _lib.ERR_INVALID_INPUT and "element type" in _lib.last_error()
    assert dec(7, Host(1024)) == _lib.ERR_INVALID_INPUT and "element type" in _lib.last_error()
    for io in (_lib.IO_F16, _lib.IO_BF16):
        assert enc(io, Host(4 * 64 * 2 - 4)) == _lib.ERR_INVALID_INPUT and "input" in _lib.last_error()
        assert dec(io, Host(4 * 64 * 2 - 4)) == _lib.ERR_INVALID_INPUT and "output" in _lib.last_error()
        # exactly count * dim * 2 bytes passes the size check and stops at the device check
        for rc in (enc(io, Host(4 * 64 * 2)), dec(io, Host(4 * 64 * 2))):
            assert rc in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
            assert "needs" not in _lib.last_error()
    assert enc(_lib.IO_F32, Host(4 * 64 * 4 - 4)) == _lib.ERR_INVALID_INPUT


def test_channel_io_entry_points_validate_type_and_sizes(lib):
    cfg = _lib.PitchChannelConfigC(64, 4, 64, 0)
    n = 100
    codes, ranges = Host(n * 32), Host(2 * 256)

    def enc(io, inp):
        return lib.pitch_enqueue_channel_encode_io(ctypes.byref(cfg), io, inp.p, inp.nbytes, 0, codes.p,
                                                   codes.nbytes, 0, ranges.p, ranges.nbytes, 0, n, None)

    def dec(io, out):
        return lib.pitch_enqueue_channel_decode_io(ctypes.byref(cfg), io, codes.p, codes.nbytes, 0, ranges.p,
                                                   ranges.nbytes, 0, out.p, out.nbytes, 0, n, None)

    assert enc(3, Host(n * 256)) == _lib.ERR_INVALID_INPUT and "element type" in _lib.last_error()
    for io in (_lib.IO_F16, _lib.IO_BF16):
        assert enc(io, Host(n * 128 - 4)) == _lib.ERR_INVALID_INPUT and "input" in _lib.last_error()
        assert dec(io, Host(n * 128 - 4)) == _lib.ERR_INVALID_INPUT and "output" in _lib.last_error()
        for rc in (enc(io, Host(n * 128)), dec(io, Host(n * 128))):
            assert rc in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
            assert "needs" not in _lib.last_error()


# ----------------------------------------------------------------------------- attention over compressed caches
def _attn_desc(nq=4, kv=2, T=100, ts=1, hs=100, scale=0.125):
    return _lib.PitchAttentionDescC(nq, kv, T, ts, hs, scale, 0)


def _attn(lib, kc, vc, desc, sizes=None, ws=None, lse=True):
    """Calls pitch_enqueue_attention_decode with host buffers sized by `sizes` (never reaching a kernel)."""
    dim = kc.dim
    nq, kv, T = desc.q_per_kv, desc.kv_heads, desc.tokens
    vecs = min((T - 1) * desc.token_stride + (kv - 1) * desc.head_stride + 1, 1 << 20)
    kcs, vcs = ((dim * kc.bits + 31) // 32) * 4, ((dim * vc.bits + 31) // 32) * 4
    need = dict(q=kv * nq * dim * 4, kcodes=vecs * kcs, kscales=vecs * 4, vcodes=vecs * vcs, vscales=vecs * 4,
                out=kv * nq * dim * 4, lse=kv * nq * 4)
    need.update(sizes or {})
    bufs = {k: Host(v) for k, v in need.items()}
    if ws is None:
        n = ctypes.c_uint64(0)
        assert lib.pitch_attention_workspace_size(ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(desc),
                                                  ctypes.byref(n)) == 0
        ws = n.value
    w = Host(ws)
    args = []
    for k in ("q", "kcodes", "kscales", "vcodes", "vscales", "out"):
        args += [bufs[k].p, bufs[k].nbytes, 0]
    args += [bufs["lse"].p, bufs["lse"].nbytes, 0] if lse else [None, 0, 0]
    return lib.pitch_enqueue_attention_decode(ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(desc), *args,
                                              w.p, w.nbytes, None)


def test_attention_workspace_size(lib):
    kc = _lib.PitchConfigC(0, 128, 4, 0)
    n = ctypes.c_uint64(0)
    sizes = []
    for T in (1, 1000, 100000):
        assert lib.pitch_attention_workspace_size(ctypes.byref(kc), ctypes.byref(kc), ctypes.byref(_attn_desc(4, 8, T)),
                                                  ctypes.byref(n)) == 0
        sizes.append(n.value)
    assert 0 < sizes[0] < sizes[1] < sizes[2]
    # at least the rotated queries and one weight per token and query head
    assert sizes[2] >= 4 * 8 * 4 * (128 + 100000)


def test_attention_validation(lib):
    k = _lib.PitchConfigC(0, 128, 4, 0)
    v = _lib.PitchConfigC(1, 128, 2, 9)
    d = _attn_desc()
    assert _attn(lib, k, _lib.PitchConfigC(0, 64, 4, 0), d, ws=1 << 20) == _lib.ERR_CONFIGURATION_MISMATCH
    assert _attn(lib, _lib.PitchConfigC(0, 256, 4, 0), _lib.PitchConfigC(0, 256, 4, 0), d, ws=1 << 20) \
        == _lib.ERR_INVALID_DIMENSION
    for bad in (_attn_desc(nq=0), _attn_desc(nq=9), _attn_desc(kv=0), _attn_desc(T=0), _attn_desc(scale=float("inf"))):
        assert _attn(lib, k, v, bad, ws=1 << 20) == _lib.ERR_INVALID_INPUT
    base = _attn(lib, k, v, d)                      # exact sizes pass every check before the device check
    assert base in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE) and "needs" not in _lib.last_error()
    # one byte short in any buffer fails the size check
    vecs = 99 + 100 + 1
    short = dict(q=2 * 4 * 128 * 4 - 4, kcodes=vecs * 64 - 4, kscales=vecs * 4 - 4, vcodes=vecs * 32 - 4,
                 vscales=vecs * 4 - 4, out=2 * 4 * 128 * 4 - 4, lse=2 * 4 * 4 - 4)
    for name, size in short.items():
        assert _attn(lib, k, v, d, sizes={name: size}) == _lib.ERR_INVALID_INPUT, name
        assert "needs" in _lib.last_error()
    n = ctypes.c_uint64(0)
    lib.pitch_attention_workspace_size(ctypes.byref(k), ctypes.byref(v), ctypes.byref(d), ctypes.byref(n))
    assert _attn(lib, k, v, d, ws=n.value - 4) == _lib.ERR_INVALID_INPUT and "workspace" in _lib.last_error()
    # lse is optional; token-major strides size the caches by the largest vector index
    assert _attn(lib, k, v, d, lse=False) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
    tm = _attn_desc(nq=1, kv=3, T=50, ts=3, hs=1)
    assert _attn(lib, k, v, tm, sizes={"kscales": (49 * 3 + 2 + 1) * 4 - 4}) == _lib.ERR_INVALID_INPUT
    small = {x: 4096 for x in ("q", "kcodes", "kscales", "vcodes", "vscales", "out", "lse")}
    assert _attn(lib, k, v, _attn_desc(T=2, ts=1 << 62, hs=1 << 62), sizes=small, ws=1 << 20) == _lib.ERR_INVALID_INPUT
    assert "overflow" in _lib.last_error()


def test_channel_append_validation(lib):
    cfg = _lib.PitchChannelConfigC(64, 4, 64, 0)
    T = 150
    inp, codes, ranges = Host(T * 256), Host(T * 32), Host(3 * 256)

    def app(total, new, io=0, r=ranges, i=inp):
        return lib.pitch_enqueue_channel_append(ctypes.byref(cfg), io, i.p, i.nbytes, 0, codes.p, codes.nbytes, 0,
                                                r.p, r.nbytes, 0, total, new, None)

    assert app(T, 0) == _lib.ERR_INVALID_INPUT
    assert app(10, 11) == _lib.ERR_INVALID_INPUT
    assert app(T, 5, io=3) == _lib.ERR_INVALID_INPUT
    assert app(T + 1, 1) == _lib.ERR_INVALID_INPUT and "needs" in _lib.last_error()      # input too small
    assert app(T, 1, r=Host(2 * 256)) == _lib.ERR_INVALID_INPUT and "ranges" in _lib.last_error()
    assert app(T, 1, io=1, i=Host(T * 128)) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
    assert "needs" not in _lib.last_error()
    assert app(T, 1) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)


def test_channel_append_16bit_odd_group_offset(lib):
    """16-bit keys with dim = 3, G = 7: the group holding the first new token starts at token 7, i.e. at byte
    7 * 3 * 2 = 42 = 2 mod 4 of the input. That derived offset needs only element alignment: the call passes
    every argument check and stops at the device lookup (no GPU here) or the device-memory check, never at
    the offset check. A caller's own input offset must still be a multiple of 4."""
    cfg = _lib.PitchChannelConfigC(3, 4, 7, 0)
    T = 12                                            # groups [0, 7) and [7, 12)
    inp, codes, ranges = Host(T * 3 * 2), Host(T * 4), Host(2 * 12)

    def app(total, new, off=0):
        return lib.pitch_enqueue_channel_append(ctypes.byref(cfg), _lib.IO_F16, inp.p, inp.nbytes, off, codes.p,
                                                codes.nbytes, 0, ranges.p, ranges.nbytes, 0, total, new, None)

    for io in (_lib.IO_F16, _lib.IO_BF16):
        rc = lib.pitch_enqueue_channel_append(ctypes.byref(cfg), io, inp.p, inp.nbytes, 0, codes.p, codes.nbytes, 0,
                                              ranges.p, ranges.nbytes, 0, T, 2, None)
        assert rc in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
        assert "offset" not in _lib.last_error() and "needs" not in _lib.last_error(), _lib.last_error()
    assert app(T - 1, 1, off=2) == _lib.ERR_INVALID_INPUT and "multiple of 4" in _lib.last_error()


def test_channel_count_bound(lib):
    """Per-channel calls take at most 2^32 - 1 tokens (the kernels count tokens and groups in 32 bits, with the
    group count formed in 64 bits); one more is refused before any size check."""
    cfg = _lib.PitchChannelConfigC(1, 2, 65536, 0)
    big = Host(1 << 12)
    rc = lib.pitch_enqueue_channel_encode(ctypes.byref(cfg), big.p, big.nbytes, 0, big.p, big.nbytes, 0, big.p,
                                          big.nbytes, 0, 2 ** 32, None)
    assert rc == _lib.ERR_INVALID_INPUT and "2^32" in _lib.last_error()
    rc = lib.pitch_enqueue_channel_decode(ctypes.byref(cfg), big.p, big.nbytes, 0, big.p, big.nbytes, 0, big.p,
                                          big.nbytes, 0, 2 ** 32, None)
    assert rc == _lib.ERR_INVALID_INPUT and "2^32" in _lib.last_error()
    # 2^32 - 1 tokens passes the count check and fails only on the (small) buffers
    rc = lib.pitch_enqueue_channel_encode(ctypes.byref(cfg), big.p, big.nbytes, 0, big.p, big.nbytes, 0, big.p,
                                          big.nbytes, 0, 2 ** 32 - 1, None)
    assert rc == _lib.ERR_INVALID_INPUT and "needs" in _lib.last_error()


def test_attention_channel_keys_validation(lib):
    kc = _lib.PitchChannelConfigC(64, 4, 64, 0)
    vc = _lib.PitchConfigC(0, 64, 4, 0)
    desc = _lib.PitchAttentionDescC(2, 2, 100, 1, 128, 0.125, 0)
    n = ctypes.c_uint64(0)
    assert lib.pitch_attention_channel_keys_workspace_size(ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(desc),
                                                           ctypes.byref(n)) == 0 and n.value > 0
    vecs = 128 + 100
    sizes = dict(q=2 * 2 * 64 * 4, kcodes=vecs * 32, kranges=4 * 256, vcodes=vecs * 32, vscales=vecs * 4,
                 out=2 * 2 * 64 * 4, lse=2 * 2 * 4)

    def call(kcfg=kc, d=desc, **over):
        sz = dict(sizes, **over)
        b = {k: Host(v) for k, v in sz.items()}
        w = Host(n.value)
        args = []
        for k in ("q", "kcodes", "kranges", "vcodes", "vscales", "out", "lse"):
            args += [b[k].p, b[k].nbytes, 0]
        return lib.pitch_enqueue_attention_decode_channel_keys(ctypes.byref(kcfg), ctypes.byref(vc), ctypes.byref(d),
                                                               *args, w.p, w.nbytes, None)

    assert call() in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE) and "needs" not in _lib.last_error()
    assert call(kcfg=_lib.PitchChannelConfigC(64, 4, 32, 0)) == _lib.ERR_INVALID_INPUT     # G not a multiple of 64
    assert "multiple of 64" in _lib.last_error()
    assert call(d=_lib.PitchAttentionDescC(2, 2, 100, 2, 128, 0.125, 0)) == _lib.ERR_INVALID_INPUT  # token stride
    assert call(d=_lib.PitchAttentionDescC(2, 2, 100, 1, 96, 0.125, 0)) == _lib.ERR_INVALID_INPUT   # head stride
    assert call(kranges=4 * 256 - 4) == _lib.ERR_INVALID_INPUT and "key ranges" in _lib.last_error()
    assert call(kcfg=_lib.PitchChannelConfigC(128, 4, 64, 0)) == _lib.ERR_CONFIGURATION_MISMATCH


def test_encode_batch_validation(lib):
    """pitch_enqueue_encode_batch checks every segment as pitch_enqueue_encode checks its buffers (sizes after the
    offsets, 4-byte offsets, count >= 1), naming the segment, before it looks for a device."""
    assert ctypes.sizeof(_lib.PitchEncodeItemC) == 80
    cfg = _lib.PitchConfigC(0, 64, 4, 0)                 # code stride 32 bytes
    bufs = []

    def items(specs):
        arr = (_lib.PitchEncodeItemC * len(specs))()
        for e, (count, ib, cb, sb, offs) in zip(arr, specs):
            i, c, s = Host(ib), Host(cb), Host(sb)
            bufs.extend((i, c, s))
            e.input, e.input_bytes, e.input_offset = i.p, ib, offs[0]
            e.codes, e.codes_bytes, e.codes_offset = c.p, cb, offs[1]
            e.scales, e.scales_bytes, e.scales_offset = s.p, sb, offs[2]
            e.count = count
        return arr

    good = (3, 3 * 256, 3 * 32, 12, (0, 0, 0))
    call = lambda arr, n=None, c=cfg, io=0: lib.pitch_enqueue_encode_batch(  # noqa: E731
        ctypes.byref(c) if c is not None else None, io, arr, len(arr) if n is None else n, None)
    assert call(items([good, good])) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
    assert "segment" not in _lib.last_error()
    assert call(items([good]), n=0) == _lib.ERR_INVALID_INPUT
    assert lib.pitch_enqueue_encode_batch(ctypes.byref(cfg), 0, None, 1, None) == _lib.ERR_INVALID_INPUT
    assert call(items([good]), c=None) == _lib.ERR_INVALID_INPUT
    assert call(items([good]), c=_lib.PitchConfigC(0, 96, 4, 0)) == _lib.ERR_INVALID_DIMENSION
    assert call(items([good]), io=3) == _lib.ERR_INVALID_INPUT
    assert call(items([good, (0, 0, 0, 0, (0, 0, 0))])) == _lib.ERR_INVALID_INPUT
    assert "segment 1" in _lib.last_error()
    assert call(items([good, good, (3, 3 * 256, 3 * 32 - 4, 12, (0, 0, 0))])) == _lib.ERR_INVALID_INPUT
    assert "codes" in _lib.last_error()
    assert call(items([(3, 3 * 256 + 8, 3 * 32, 12, (6, 0, 0))])) == _lib.ERR_INVALID_INPUT   # misaligned
    assert call(items([(3, 3 * 256, 3 * 32, 16, (0, 0, 8))])) == _lib.ERR_INVALID_INPUT       # 8 bytes left
    assert call(items([(3, 3 * 128, 3 * 32, 12, (0, 0, 0))]), io=1) in (_lib.ERR_INVALID_INPUT,
                                                                       _lib.ERR_DEVICE_UNAVAILABLE)
    assert "segment" not in _lib.last_error() and "needs" not in _lib.last_error()


def test_decode_batch_validation(lib):
    """pitch_enqueue_decode_batch checks every segment as pitch_enqueue_decode checks its buffers (sizes after the
    offsets, 4-byte offsets, count >= 1), naming the segment, before it looks for a device."""
    assert ctypes.sizeof(_lib.PitchDecodeItemC) == 80
    cfg = _lib.PitchConfigC(0, 64, 4, 0)                 # code stride 32 bytes
    bufs = []

    def items(specs):
        arr = (_lib.PitchDecodeItemC * len(specs))()
        for e, (count, cb, sb, ob, offs) in zip(arr, specs):
            c, s, o = Host(cb), Host(sb), Host(ob)
            bufs.extend((c, s, o))
            e.codes, e.codes_bytes, e.codes_offset = c.p, cb, offs[0]
            e.scales, e.scales_bytes, e.scales_offset = s.p, sb, offs[1]
            e.output, e.output_bytes, e.output_offset = o.p, ob, offs[2]
            e.count = count
        return arr

    good = (3, 3 * 32, 12, 3 * 256, (0, 0, 0))
    call = lambda arr, n=None, c=cfg, io=0: lib.pitch_enqueue_decode_batch(  # noqa: E731
        ctypes.byref(c) if c is not None else None, io, arr, len(arr) if n is None else n, None)
    assert call(items([good, good])) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)
    assert "segment" not in _lib.last_error()
    assert call(items([good]), n=0) == _lib.ERR_INVALID_INPUT
    assert lib.pitch_enqueue_decode_batch(ctypes.byref(cfg), 0, None, 1, None) == _lib.ERR_INVALID_INPUT
    assert call(items([good]), c=None) == _lib.ERR_INVALID_INPUT
    assert call(items([good]), c=_lib.PitchConfigC(0, 96, 4, 0)) == _lib.ERR_INVALID_DIMENSION
    assert call(items([good]), io=3) == _lib.ERR_INVALID_INPUT
    assert call(items([good, (0, 0, 0, 0, (0, 0, 0))])) == _lib.ERR_INVALID_INPUT
    assert "segment 1" in _lib.last_error()
    assert call(items([good, good, (3, 3 * 32, 12, 3 * 256 - 4, (0, 0, 0))])) == _lib.ERR_INVALID_INPUT
    assert "output" in _lib.last_error()
    assert call(items([(3, 3 * 32 + 8, 12, 3 * 256, (6, 0, 0))])) == _lib.ERR_INVALID_INPUT   # misaligned
    assert call(items([(3, 3 * 32, 16, 3 * 256, (0, 8, 0))])) == _lib.ERR_INVALID_INPUT       # 8 bytes left
    assert call(items([(3, 3 * 32, 12, 3 * 128, (0, 0, 0))]), io=1) in (_lib.ERR_INVALID_INPUT,
                                                                       _lib.ERR_DEVICE_UNAVAILABLE)
    assert "segment" not in _lib.last_error() and "needs" not in _lib.last_error()


def test_attention_key_bias_validation(lib):
    """The key-bias attention entry: null key bias, a head count other than the call's KV heads and RoPE tables
    too short for first_position + tokens rows are rejected before any device work."""
    kc = _lib.PitchConfigC(0, 64, 4, 0)
    T, kv, nq, d = 100, 2, 2, 64
    desc = _lib.PitchAttentionDescC(nq, kv, T, kv, 1, 0.125, 0)
    n = ctypes.c_uint64(0)
    assert lib.pitch_attention_workspace_size(ctypes.byref(kc), ctypes.byref(kc), ctypes.byref(desc),
                                              ctypes.byref(n)) == 0
    vecs = T * kv
    bufs = [Host(x) for x in (kv * nq * d * 4, vecs * 32, vecs * 4, vecs * 32, vecs * 4, kv * nq * d * 4,
                              kv * nq * 4)]
    w = Host(n.value)
    bias, cos, sin = Host(kv * d * 4), Host((T + 10) * d * 4), Host((T + 10) * d * 4)

    def call(first=0, heads=kv, kb=True, tb=(T + 10) * d * 4):
        k = _lib.PitchKeyBiasC(bias.p, kv * d * 4, cos.p, sin.p, tb, first, heads, 0)
        args = []
        for b in bufs:
            args += [b.p, b.nbytes, 0]
        return lib.pitch_enqueue_attention_decode_key_bias(ctypes.byref(kc), ctypes.byref(kc), ctypes.byref(desc),
                                                           ctypes.byref(k) if kb else None, *args, w.p, w.nbytes,
                                                           None)

    assert call() in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE) and "positions" not in _lib.last_error()
    assert call(kb=False) == _lib.ERR_INVALID_INPUT
    assert call(heads=1) == _lib.ERR_INVALID_INPUT and "KV heads" in _lib.last_error()
    assert call(first=10) in (_lib.ERR_INVALID_INPUT, _lib.ERR_DEVICE_UNAVAILABLE)   # exactly T rows left
    assert "positions" not in _lib.last_error()
    assert call(first=11) == _lib.ERR_INVALID_INPUT and "positions" in _lib.last_error()
    assert call(tb=T * d * 4 - 4) == _lib.ERR_INVALID_INPUT


def test_calibration_library_exports_and_rejects_bad_arguments(built_library):
    """libpitch_calib.so (bench.py's same-traffic streams) is built beside the codec and exports its two entry
    points; arguments out of range return -1 before any HIP call (null pointers, a unit that is not a whole number
    of pieces, an unknown piece size or launch mode)."""
    from pitch_amd.build import CALIB_LIB
    if not CALIB_LIB.exists():
        from pitch_amd.build import build
        build()
    calib = ctypes.CDLL(str(CALIB_LIB))
    st, ss = calib.pitch_calib_stream, calib.pitch_calib_stream_store
    st.restype = ss.restype = ctypes.c_int
    st.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                   ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    ss.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                   ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) & ~15
    assert st(None, p, 4, 512, 13, 128, 768, 1, None) == -1
    assert st(p, None, 4, 512, 13, 128, 768, 1, None) == -1
    assert st(p, p, 0, 512, 13, 128, 768, 1, None) == -1      # no units
    assert st(p, p, 4, 500, 13, 128, 768, 1, None) == -1      # not whole pieces
    assert st(p, p, 4, 96, 13, 96, 768, 1, None) == -1        # unknown piece size
    assert st(p + 4, p, 4, 512, 13, 128, 768, 1, None) == -1  # input not 16-byte aligned
    assert ss(None, p, 4, 512, 13, 128, 2, 2048, 1, None) == -1
    assert ss(p, p, 4, 512, 13, 128, 3, 2048, 1, None) == -1  # unknown launch mode
    assert ss(p, p + 4, 4, 512, 13, 128, 2, 2048, 1, None) == -1  # output not 16-byte aligned
    assert ss(p, p, 4, 512, 13, 32, 2, 2048, 1, None) == -1   # unknown piece size
