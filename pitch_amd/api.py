"""Host-side operator surface of the MI355X codec, mirroring SwiftCham/PITCH's public API.

Types and methods keep the reference's names and meaning (Sources/PITCH/PITCH.swift, PerChannel.swift,
Models/*.swift): ``QuantConfig``, ``ChannelQuantConfig``, ``CompressedBatch``, ``ChannelCompressedBlock``,
``PITCH.config/encode/decode/enqueueEncode/enqueueDecode`` and the per-channel forms. Tensors are
PyTorch-ROCm device tensors; the GPU-resident ``enqueue*`` forms take caller-owned tensors with byte
offsets and launch on a HIP stream without waiting, like the reference's command-buffer forms. The array
forms copy, launch, wait and copy back.

All arithmetic runs in libpitch_amd.so (hand-written HIP kernels); this module only validates, allocates
and calls through the C ABI.
"""
from __future__ import annotations

import base64
import ctypes
import math
import enum
import json
from dataclasses import dataclass, field

import numpy as np

from . import _lib

DEFAULT_SEED = 0x50495443                 # PITCH.defaultSeed (Sources/PITCH/PITCH.swift:18)


# ----------------------------------------------------------------------------------------- errors
class PITCHError(Exception):
    """Base of the error enum PITCHError (Sources/PITCH/Core/PITCHError.swift:10-19)."""


class InvalidInput(PITCHError, ValueError):
    pass


class InvalidBitWidth(PITCHError, ValueError):
    def __init__(self, bits, message: str | None = None):
        super().__init__(message or f"Invalid bit width {bits}. Must be in 2...8.")
        self.bits = bits


class InvalidDimension(PITCHError, ValueError):
    def __init__(self, dim, message: str | None = None):
        super().__init__(message or f"Invalid dimension {dim}. Must be a power of two in [2, 1024].")
        self.dim = dim


class ConfigurationMismatch(PITCHError):
    pass


class EncodingFailed(PITCHError, RuntimeError):
    pass


class DecodingFailed(PITCHError, RuntimeError):
    pass


class DeviceUnavailable(PITCHError, RuntimeError):
    """No usable GPU or HIP library (the reference's metalNotSupported)."""


def _lib_or_raise():
    try:
        return _lib.load()
    except (RuntimeError, OSError) as e:
        raise DeviceUnavailable(str(e)) from e


def _raise_for(rc: int, what: str = "") -> None:
    if rc == _lib.PITCH_OK:
        return
    msg = _lib.last_error() or what
    if rc == _lib.ERR_INVALID_BIT_WIDTH:
        raise InvalidBitWidth(None, msg)
    if rc == _lib.ERR_INVALID_DIMENSION:
        raise InvalidDimension(None, msg)
    raise {
        _lib.ERR_INVALID_INPUT: InvalidInput,
        _lib.ERR_CONFIGURATION_MISMATCH: ConfigurationMismatch,
        _lib.ERR_ENCODING_FAILED: EncodingFailed,
        _lib.ERR_DECODING_FAILED: DecodingFailed,
        _lib.ERR_DEVICE_UNAVAILABLE: DeviceUnavailable,
    }.get(rc, PITCHError)(msg)


# ----------------------------------------------------------------------------------------- configs
class QuantMethod(str, enum.Enum):
    """Sources/PITCH/Models/QuantMethod.swift:8-11."""
    turboQuant = "turboQuant"
    polarQuant = "polarQuant"

    @property
    def code(self) -> int:
        return 0 if self is QuantMethod.turboQuant else 1


def _method(m) -> QuantMethod:
    try:
        return m if isinstance(m, QuantMethod) else QuantMethod(m)
    except ValueError:
        raise InvalidInput(f"unknown method {m!r}") from None


@dataclass(frozen=True)
class QuantConfig:
    """Everything needed to interpret a batch of compressed vectors (Models/QuantConfig.swift:11-60)."""
    method: QuantMethod
    dim: int
    bits: int
    seed: int = DEFAULT_SEED

    supportedBits = range(2, 9)
    maxDimension = 1024
    maxInputMagnitude = 1e17

    def __post_init__(self):
        object.__setattr__(self, "method", _method(self.method))
        if not isinstance(self.dim, (int, np.integer)) or not isinstance(self.bits, (int, np.integer)):
            raise InvalidInput("dim and bits must be integers")
        if not (0 <= int(self.seed) <= 0xFFFFFFFF):
            raise InvalidInput(f"seed {self.seed} must fit in 32 bits")
        if int(self.dim) < 0 or int(self.dim) > 0xFFFFFFFF:
            raise InvalidDimension(self.dim)
        if int(self.bits) < 0 or int(self.bits) > 0xFFFFFFFF:
            raise InvalidBitWidth(self.bits)
        c = _lib.PitchConfigC()
        cs = ctypes.c_uint32()
        _raise_for(_lib_or_raise().pitch_config(self.method.code, int(self.dim), int(self.bits),
                                                int(self.seed), ctypes.byref(c), ctypes.byref(cs)))
        object.__setattr__(self, "dim", int(self.dim))
        object.__setattr__(self, "bits", int(self.bits))
        object.__setattr__(self, "seed", int(self.seed))
        object.__setattr__(self, "_cs", int(cs.value))
        object.__setattr__(self, "_cstruct", c)  # the C ABI's view, built once (the config is immutable)

    def _c(self) -> _lib.PitchConfigC:
        return self._cstruct

    @property
    def codeStride(self) -> int:
        """Bytes of packed codes per vector: ceil(dim * bits / 32) * 4 (QuantConfig.swift:47)."""
        return self._cs

    @property
    def bytesPerVector(self) -> int:
        return self.codeStride + 4

    @property
    def bitsPerCoordinate(self) -> float:
        return self.bytesPerVector * 8 / self.dim

    @property
    def compressionRatio(self) -> float:
        return 32.0 / self.bitsPerCoordinate

    @property
    def compressionRatioVsFloat16(self) -> float:
        return 16.0 / self.bitsPerCoordinate

    def to_dict(self) -> dict:
        return {"method": self.method.value, "dim": self.dim, "bits": self.bits, "seed": self.seed}


@dataclass(frozen=True)
class ChannelQuantConfig:
    """Per-channel (KIVI-style) key configuration (Sources/PITCH/PerChannel.swift:15-70)."""
    dim: int
    bits: int
    groupSize: int = 64

    supportedBits = range(2, 9)
    maxDimension = 1024
    supportedGroupSizes = range(1, 65537)
    defaultGroupSize = 64
    maxInputMagnitude = 65504.0

    def __post_init__(self):
        for name in ("dim", "bits", "groupSize"):
            v = getattr(self, name)
            if not isinstance(v, (int, np.integer)) or not (0 <= int(v) <= 0xFFFFFFFF):
                raise InvalidInput(f"{name} {v!r} must be a non-negative integer")
            object.__setattr__(self, name, int(v))
        c = _lib.PitchChannelConfigC()
        cs, rs = ctypes.c_uint32(), ctypes.c_uint32()
        _raise_for(_lib_or_raise().pitch_channel_config(self.dim, self.bits, self.groupSize, ctypes.byref(c),
                                                        ctypes.byref(cs), ctypes.byref(rs)))
        object.__setattr__(self, "_cs", int(cs.value))
        object.__setattr__(self, "_rs", int(rs.value))
        object.__setattr__(self, "_cstruct", c)

    def _c(self) -> _lib.PitchChannelConfigC:
        return self._cstruct

    @property
    def codeStride(self) -> int:
        return self._cs

    @property
    def rangeStride(self) -> int:
        """Bytes of fp16 ranges per group: dim minima then dim maxima (PerChannel.swift:58)."""
        return self._rs

    def groupCount(self, tokens: int) -> int:
        return (int(tokens) + self.groupSize - 1) // self.groupSize

    @property
    def bitsPerCoordinate(self) -> float:
        return self.codeStride * 8 / self.dim + self.rangeStride * 8 / (self.dim * self.groupSize)

    @property
    def compressionRatio(self) -> float:
        return 32.0 / self.bitsPerCoordinate

    @property
    def compressionRatioVsFloat16(self) -> float:
        return 16.0 / self.bitsPerCoordinate

    def to_dict(self) -> dict:
        return {"dim": self.dim, "bits": self.bits, "groupSize": self.groupSize}


# ----------------------------------------------------------------------------------------- containers
def half_to_float(h: int) -> float:
    """IEEE fp16 bits to float (PerChannel.swift:171-180)."""
    return float(np.array([h], dtype=np.uint16).view(np.float16)[0])


@dataclass
class CompressedBatch:
    """Vectors sharing one QuantConfig: codes of vector i at bytes [i*codeStride, (i+1)*codeStride), scale
    scales[i] (Sources/PITCH/Models/CompressedBatch.swift:13-121)."""
    config: QuantConfig
    codes: bytes
    scales: np.ndarray
    _checked: bool = field(default=True, repr=False, compare=False)

    headerByteCount = 16
    formatVersion = 3

    def __post_init__(self):
        self.codes = bytes(self.codes)
        self.scales = np.ascontiguousarray(np.asarray(self.scales, dtype=np.float32).reshape(-1))
        if self._checked:
            self.validate()

    def __eq__(self, other):
        return (isinstance(other, CompressedBatch) and self.config == other.config and self.codes == other.codes
                and np.array_equal(self.scales.view(np.uint32), other.scales.view(np.uint32)))

    @property
    def count(self) -> int:
        return int(self.scales.shape[0])

    def validate(self) -> None:
        """CompressedBatch.swift:35-47."""
        if self.count == 0:
            raise InvalidInput("a batch must contain at least one vector")
        expected = self.count * self.config.codeStride
        if len(self.codes) != expected:
            raise InvalidInput(f"codes is {len(self.codes)} bytes; expected {expected} for {self.count} vectors")
        if not (np.isfinite(self.scales).all() and (self.scales >= 0).all()):
            raise InvalidInput("scales must be finite and non-negative")

    def append(self, other: "CompressedBatch") -> None:
        if other.config != self.config:
            raise ConfigurationMismatch("cannot append a batch with a different config")
        self.codes = self.codes + other.codes
        self.scales = np.concatenate([self.scales, other.scales])

    def vectors(self, rng) -> "CompressedBatch":
        """The vectors in range(lo, hi) as a new batch (CompressedBatch.swift:59-70)."""
        lo, hi = (rng.start, rng.stop) if isinstance(rng, (range, slice)) else rng
        lo = 0 if lo is None else lo
        hi = self.count if hi is None else hi
        if lo < 0 or hi > self.count or hi <= lo:
            raise InvalidInput(f"range {lo}..<{hi} is outside 0..<{self.count}")
        s = self.config.codeStride
        return CompressedBatch(self.config, self.codes[lo * s:hi * s], self.scales[lo:hi].copy(), _checked=False)

    @property
    def payloadByteCount(self) -> int:
        return len(self.codes)

    @property
    def sideInformationByteCount(self) -> int:
        return self.count * 4 + self.headerByteCount

    @property
    def storedByteCount(self) -> int:
        return self.payloadByteCount + self.sideInformationByteCount

    @property
    def originalByteCount(self) -> int:
        return self.count * self.config.dim * 4

    @property
    def compressionRatio(self) -> float:
        return self.originalByteCount / self.storedByteCount

    @property
    def compressionRatioVsFloat16(self) -> float:
        return self.compressionRatio / 2

    @property
    def bitsPerCoordinate(self) -> float:
        return self.storedByteCount * 8 / (self.count * self.config.dim)

    # Codable form v3 (CompressedBatch.swift:95-121): {"formatVersion", "config", "codes" (base64), "scales"}
    def to_json(self) -> str:
        return json.dumps({"formatVersion": self.formatVersion, "config": self.config.to_dict(),
                           "codes": base64.b64encode(self.codes).decode(),
                           "scales": [float(s) for s in self.scales]})

    @classmethod
    def from_json(cls, text: str) -> "CompressedBatch":
        """Decodes a CompressedBatch as Swift's JSONDecoder does for the reference's CodingKeys
        (CompressedBatch.swift:95-121, QuantConfig.swift:37-45): any key order, `codes` strict base64, `scales` a
        number array, `config` {method, dim, bits, seed}; the config and sizes are validated."""
        obj = _json_object(text)
        _check_version(obj, cls.formatVersion, "")
        c = _json_field(obj, "config", dict)
        cfg = QuantConfig(_json_field(c, "method", str), _json_int(c, "dim"), _json_int(c, "bits"),
                          _json_int(c, "seed"))
        return cls(cfg, _json_base64(obj, "codes"), _json_numbers(obj, "scales", np.float32))


@dataclass
class ChannelCompressedBlock:
    """Per-channel compressed keys: codes per token plus fp16 ranges [group][min row][max row]
    (Sources/PITCH/PerChannel.swift:72-168)."""
    config: ChannelQuantConfig
    codes: bytes
    ranges: np.ndarray
    _checked: bool = field(default=True, repr=False, compare=False)

    headerByteCount = 16
    formatVersion = 1

    def __post_init__(self):
        self.codes = bytes(self.codes)
        self.ranges = np.ascontiguousarray(np.asarray(self.ranges, dtype=np.uint16).reshape(-1))
        if self._checked:
            self.validate()

    def __eq__(self, other):
        return (isinstance(other, ChannelCompressedBlock) and self.config == other.config
                and self.codes == other.codes and np.array_equal(self.ranges, other.ranges))

    @property
    def count(self) -> int:
        return len(self.codes) // self.config.codeStride

    @property
    def groupCount(self) -> int:
        return self.config.groupCount(self.count)

    def validate(self) -> None:
        """PerChannel.swift:94-113."""
        cs = self.config.codeStride
        if len(self.codes) == 0 or len(self.codes) % cs != 0:
            raise InvalidInput(f"codes is {len(self.codes)} bytes; expected a positive multiple of {cs}")
        expected = self.groupCount * 2 * self.config.dim
        if self.ranges.shape[0] != expected:
            raise InvalidInput(f"ranges has {self.ranges.shape[0]} values; expected {expected} for {self.count} tokens")
        r = self.ranges.view(np.float16).astype(np.float32).reshape(self.groupCount, 2, self.config.dim)
        lo, hi = r[:, 0], r[:, 1]
        bad = ~(np.isfinite(lo) & np.isfinite(hi) & (lo <= hi))
        if bad.any():
            g, ch = map(int, np.argwhere(bad)[0])
            raise InvalidInput(f"group {g} channel {ch}: range [{lo[g, ch]}, {hi[g, ch]}] is invalid")

    def range(self, group: int, channel: int) -> tuple[float, float]:
        d = self.config.dim
        return (half_to_float(self.ranges[group * 2 * d + channel]),
                half_to_float(self.ranges[group * 2 * d + d + channel]))

    def append(self, other: "ChannelCompressedBlock") -> None:
        if other.config != self.config:
            raise ConfigurationMismatch("cannot append a block with a different config")
        if self.count % self.config.groupSize != 0:
            raise InvalidInput(f"cannot append after a partial group ({self.count} tokens, group size "
                               f"{self.config.groupSize})")
        self.codes = self.codes + other.codes
        self.ranges = np.concatenate([self.ranges, other.ranges])

    @property
    def payloadByteCount(self) -> int:
        return len(self.codes)

    @property
    def sideInformationByteCount(self) -> int:
        return self.ranges.shape[0] * 2 + self.headerByteCount

    @property
    def storedByteCount(self) -> int:
        return self.payloadByteCount + self.sideInformationByteCount

    @property
    def originalByteCount(self) -> int:
        return self.count * self.config.dim * 4

    @property
    def compressionRatio(self) -> float:
        return self.originalByteCount / self.storedByteCount

    @property
    def compressionRatioVsFloat16(self) -> float:
        return self.compressionRatio / 2

    @property
    def bitsPerCoordinate(self) -> float:
        return self.storedByteCount * 8 / (self.count * self.config.dim)

    def to_json(self) -> str:
        return json.dumps({"formatVersion": self.formatVersion, "config": self.config.to_dict(),
                           "codes": base64.b64encode(self.codes).decode(),
                           "ranges": [int(r) for r in self.ranges]})

    @classmethod
    def from_json(cls, text: str) -> "ChannelCompressedBlock":
        """Decodes a ChannelCompressedBlock as Swift's JSONDecoder does for the reference's CodingKeys
        (PerChannel.swift:143-168, :45-52): `codes` strict base64, `ranges` an array of 16-bit integers, `config`
        {dim, bits, groupSize}."""
        obj = _json_object(text)
        _check_version(obj, cls.formatVersion, "per-channel ")
        c = _json_field(obj, "config", dict)
        cfg = ChannelQuantConfig(_json_int(c, "dim"), _json_int(c, "bits"), _json_int(c, "groupSize"))
        return cls(cfg, _json_base64(obj, "codes"), _json_numbers(obj, "ranges", np.uint16))


# JSON decoding with the reference's failure modes (Swift's DecodingError becomes InvalidInput here)
def _json_object(text: str) -> dict:
    try:
        obj = json.loads(text)
    except (ValueError, TypeError) as e:
        raise InvalidInput(f"not a JSON document: {e}") from e
    if not isinstance(obj, dict):
        raise InvalidInput("a container is a JSON object")
    return obj


def _json_field(obj: dict, key: str, kind):
    if key not in obj:
        raise InvalidInput(f"missing key '{key}'")
    v = obj[key]
    if not isinstance(v, kind) or isinstance(v, bool):
        raise InvalidInput(f"'{key}' has the wrong type")
    return v


def _json_int(obj: dict, key: str) -> int:
    v = _json_field(obj, key, (int, float))
    if isinstance(v, float) and not v.is_integer():
        raise InvalidInput(f"'{key}' is not an integer")
    return int(v)


def _check_version(obj: dict, version: int, what: str) -> None:
    v = _json_int(obj, "formatVersion")
    if v != version:
        raise InvalidInput(f"Unsupported PITCH {what}format version {v}; expected {version}")


def _json_base64(obj: dict, key: str) -> bytes:
    try:
        return base64.b64decode(_json_field(obj, key, str), validate=True)
    except ValueError as e:   # binascii.Error
        raise InvalidInput(f"'{key}' is not valid base64") from e


def _json_numbers(obj: dict, key: str, dtype) -> np.ndarray:
    v = _json_field(obj, key, list)
    if not all(isinstance(x, (int, float)) and not isinstance(x, bool) for x in v):
        raise InvalidInput(f"'{key}' must be an array of numbers")
    if dtype == np.uint16 and not all(float(x).is_integer() and 0 <= x <= 0xFFFF for x in v):
        raise InvalidInput(f"'{key}' must hold 16-bit unsigned integers")
    return np.array(v, dtype=np.float64).astype(dtype) if dtype != np.uint16 else np.array(v, dtype=np.uint16)


# ----------------------------------------------------------------------------------------- torch plumbing
def _torch():
    import torch
    return torch


def _buf(t, name: str):
    """(pointer, byte length) of a contiguous device tensor used as a raw buffer."""
    try:
        if t.is_cuda and t.is_contiguous():
            return t.data_ptr(), t.nbytes
    except AttributeError:
        pass
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise InvalidInput(f"{name} must be a torch tensor")
    if not t.is_cuda:
        raise InvalidInput(f"{name} buffer is not device memory")
    if not t.is_contiguous():
        raise InvalidInput(f"{name} buffer must be contiguous")
    return t.data_ptr(), t.numel() * t.element_size()


_IO_NAMES = {"float32": _lib.IO_F32, "float16": _lib.IO_F16, "bfloat16": _lib.IO_BF16}


def _io_type(t, element_type=None) -> int:
    """Element type code (PITCH_IO_*) of an uncompressed buffer: element_type when given (a torch dtype or
    "float32" / "float16" / "bfloat16"), else the tensor's own dtype when it is float16 or bfloat16, else
    float32 (a raw byte buffer holds float32 values, as in the reference's untyped buffers)."""
    torch = _torch()
    if element_type is None:
        return {torch.float16: _lib.IO_F16, torch.bfloat16: _lib.IO_BF16}.get(t.dtype, _lib.IO_F32)
    name = str(element_type).replace("torch.", "")
    if name not in _IO_NAMES:
        raise InvalidInput(f"element type {element_type} is not float32, float16 or bfloat16")
    return _IO_NAMES[name]


def _stream_handle(stream, device=None):
    """HIP stream handle: the given stream (an int handle or a torch stream), else torch's current stream of
    device (read with the raw query when torch has it: a fraction of a microsecond instead of about two)."""
    torch = _torch()
    if stream is None:
        raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if raw is not None:
            idx = device.index if device is not None and device.index is not None else torch.cuda.current_device()
            return raw(idx)
        return torch.cuda.current_stream(device).cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _validate_values(x, limit: float, what: str) -> None:
    """PITCH.validateValues (PITCH.swift:172-181) / validateChannelValues (PerChannel.swift:273-282)."""
    torch = _torch()
    if isinstance(x, torch.Tensor):
        finite = bool(torch.isfinite(x).all())
        largest = float(x.abs().max()) if finite and x.numel() else 0.0
    else:
        finite = bool(np.isfinite(x).all())
        largest = float(np.abs(x).max()) if finite and x.size else 0.0
    if not finite:
        raise InvalidInput("input contains NaN or infinity")
    if largest > limit:
        raise InvalidInput(f"input magnitude {largest} exceeds {limit}; {what}")


@dataclass
class KeyBias:
    """RoPE'd key-projection bias removed before encoding and restored after decoding (mechanism_eval.py:88-116):
    bias [heads][dim], cos and sin [positions][dim] fp32 device tensors (the model's own rotary tables), the
    position of the call's first token and the KV heads per token of a token-major cache."""
    bias: object
    cos: object
    sin: object
    firstPosition: int = 0
    heads: int = 1

    def _c(self) -> _lib.PitchKeyBiasC:
        bp, bb = _buf(self.bias, "key bias")
        cp, cb = _buf(self.cos, "RoPE cos")
        sp, sb = _buf(self.sin, "RoPE sin")
        if cb != sb:
            raise InvalidInput("RoPE cos and sin tables differ in size")
        if not isinstance(self.firstPosition, (int, np.integer)) or self.firstPosition < 0:
            raise InvalidInput(f"firstPosition {self.firstPosition} must be a non-negative integer")
        return _lib.PitchKeyBiasC(bp, bb, cp, sp, cb, int(self.firstPosition), int(self.heads), 0)


# ----------------------------------------------------------------------------------------- PITCH
class PITCH:
    """Public entry point (Sources/PITCH/PITCH.swift:15-189 and the PerChannel extension :182-290)."""

    defaultSeed = DEFAULT_SEED
    _shared: "PITCH | None" = None

    def __init__(self, seed: int = DEFAULT_SEED, device=None):
        if not (0 <= int(seed) <= 0xFFFFFFFF):
            raise InvalidInput(f"seed {seed} must fit in 32 bits")
        self.seed = int(seed)
        self._lib = _lib_or_raise()
        torch = _torch()
        if device is None:
            if not torch.cuda.is_available():
                raise DeviceUnavailable("no HIP device is available")
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise DeviceUnavailable(f"{device} is not a HIP device")

    @classmethod
    def shared(cls) -> "PITCH":
        if cls._shared is None:
            cls._shared = cls()
        return cls._shared

    def config(self, method, dim: int, bits: int) -> QuantConfig:
        return QuantConfig(method, dim, bits, self.seed)

    def channelConfig(self, dim: int, bits: int, groupSize: int = 64) -> ChannelQuantConfig:
        return ChannelQuantConfig(dim, bits, groupSize)

    # ---- helpers
    def _on_device(self, x, name="input"):
        """Flat device copy of the vectors, keeping a float16 or bfloat16 tensor's (or float16 array's) type."""
        torch = _torch()
        if isinstance(x, torch.Tensor):
            t = x.detach()
            if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
                raise InvalidInput(f"{name} must be float32, float16 or bfloat16")
            return t.to(self.device).contiguous().reshape(-1)
        a = np.asarray(x)
        a = a.reshape(-1) if a.dtype == np.float16 else np.asarray(a, dtype=np.float32).reshape(-1)
        if not (a.flags.c_contiguous and a.flags.writeable):
            a = a.copy()
        return torch.from_numpy(a).to(self.device)

    def _guard(self, fn, failure):
        torch = _torch()
        with torch.cuda.device(self.device):
            try:
                out = fn()
                torch.cuda.current_stream(self.device).synchronize()
                return out
            except PITCHError:
                raise
            except RuntimeError as e:
                raise failure(str(e)) from e

    # ---- array API (PITCH.swift:68-132)
    def encode(self, vectors, dim: int | None = None, bits: int | None = None, method=None,
               seed: int | None = None, config: QuantConfig | None = None) -> CompressedBatch:
        """Compresses len(vectors) / dim contiguous vectors; without dim, one vector (PITCH.swift:68-104)."""
        torch = _torch()
        n = int(vectors.numel()) if isinstance(vectors, torch.Tensor) else int(np.asarray(vectors).size)
        if config is None:
            if bits is None or method is None:
                raise InvalidInput("encode needs a config or bits and method")
            config = QuantConfig(method, n if dim is None else dim, bits, self.seed if seed is None else seed)
        if n == 0 or n % config.dim != 0:
            raise InvalidInput(f"{n} floats is not a whole number of {config.dim}-dim vectors")
        _validate_values(vectors if isinstance(vectors, torch.Tensor) else np.asarray(vectors, dtype=np.float32),
                         QuantConfig.maxInputMagnitude, "the kernels' float32 sum of squares would overflow")
        count = n // config.dim

        def run():
            x = self._on_device(vectors)
            codes = torch.empty(count * config.codeStride, dtype=torch.uint8, device=self.device)
            scales = torch.empty(count, dtype=torch.float32, device=self.device)
            self.enqueueEncode(x, codes, scales, count, config)
            return codes, scales

        codes, scales = self._guard(run, EncodingFailed)
        return CompressedBatch(config, codes.cpu().numpy().tobytes(), scales.cpu().numpy(), _checked=False)

    def decode(self, batch: CompressedBatch) -> np.ndarray:
        """Reconstructs every vector of the batch, contiguously (PITCH.swift:107-115)."""
        torch = _torch()
        out = torch.empty(batch.count * batch.config.dim, dtype=torch.float32, device=self.device)
        self.decode_into(batch, out, 0)
        return out.cpu().numpy()

    def decode_into(self, batch: CompressedBatch, buffer, offset: int = 0) -> None:
        """Reconstructs the batch into a device buffer at byte offset, then waits (PITCH.swift:118-132)."""
        torch = _torch()
        batch.validate()

        def run():
            codes = torch.from_numpy(np.frombuffer(batch.codes, dtype=np.uint8).copy()).to(self.device)
            scales = torch.from_numpy(batch.scales.copy()).to(self.device)
            self.enqueueDecode(codes, scales, buffer, batch.count, batch.config, outputOffset=offset)

        self._guard(run, DecodingFailed)

    # ---- GPU-resident API (PITCH.swift:144-165)
    def enqueueEncode(self, input, codes, scales, count: int, config: QuantConfig, inputOffset: int = 0,
                      codesOffset: int = 0, scalesOffset: int = 0, stream=None, elementType=None,
                      keyBias: KeyBias | None = None) -> None:
        """Launches encoding of count vectors; results are valid once the stream reaches this point. The input's
        element type is elementType, else the tensor's dtype when float16/bfloat16, else float32. With keyBias
        (float32 only) the vectors x - R_t b are encoded."""
        ip, ib = _buf(input, "input")
        cp, cb = _buf(codes, "codes")
        sp, sb = _buf(scales, "scales")
        _check_offsets(inputOffset, codesOffset, scalesOffset)
        io = _io_type(input, elementType)
        args = (ip, ib, inputOffset, cp, cb, codesOffset, sp, sb, scalesOffset, _count(count),
                _stream_handle(stream, self.device))
        if keyBias is not None:
            if io != _lib.IO_F32:
                raise InvalidInput("key-bias removal takes float32 vectors")
            rc = self._lib.pitch_enqueue_encode_key_bias(ctypes.byref(config._c()), ctypes.byref(keyBias._c()), *args)
        elif io == _lib.IO_F32:
            rc = self._lib.pitch_enqueue_encode(ctypes.byref(config._c()), *args)
        else:
            rc = self._lib.pitch_enqueue_encode_io(ctypes.byref(config._c()), io, *args)
        _raise_for(rc)

    def enqueueEncodeBatch(self, items, config: QuantConfig, stream=None, elementType=None) -> None:
        """Encodes independent segments with one configuration in one call (pitch_enqueue_encode_batch), with
        the same results as one enqueueEncode per segment. items: a sequence of (input, codes, scales, count)
        or (input, codes, scales, count, inputOffset, codesOffset, scalesOffset); every input has the element
        type elementType, else the first input's, chosen as for enqueueEncode. For the per-token append across
        many layers' caches (README.md:65-71 appends with one enqueueEncode per cache); EncodeBatch keeps the
        segment table between calls."""
        items = list(items)
        if not items:
            raise InvalidInput("a batch needs at least one segment")
        io = _io_type(items[0][0], elementType)
        arr = (_lib.PitchEncodeItemC * len(items))()
        for i, it in enumerate(items):
            if len(it) not in (4, 7):
                raise InvalidInput("a segment is (input, codes, scales, count[, inputOffset, codesOffset, "
                                   "scalesOffset])")
            offs = it[4:] if len(it) == 7 else (0, 0, 0)
            _check_offsets(*offs)
            if _io_type(it[0], elementType) != io:
                raise InvalidInput("every segment's input must have the batch's element type")
            e = arr[i]
            e.input, e.input_bytes = _buf(it[0], "input")
            e.codes, e.codes_bytes = _buf(it[1], "codes")
            e.scales, e.scales_bytes = _buf(it[2], "scales")
            e.input_offset, e.codes_offset, e.scales_offset = (int(o) for o in offs)
            e.count = _count(it[3])
        _raise_for(self._lib.pitch_enqueue_encode_batch(ctypes.byref(config._c()), io, arr, len(items),
                                                        _stream_handle(stream, self.device)))

    def enqueueDecode(self, codes, scales, output, count: int, config: QuantConfig, codesOffset: int = 0,
                      scalesOffset: int = 0, outputOffset: int = 0, stream=None, elementType=None,
                      keyBias: KeyBias | None = None) -> None:
        """Launches decoding of count vectors into output, whose element type is chosen as for enqueueEncode.
        With keyBias (float32 only) R_t b is added back."""
        cp, cb = _buf(codes, "codes")
        sp, sb = _buf(scales, "scales")
        op, ob = _buf(output, "output")
        _check_offsets(codesOffset, scalesOffset, outputOffset)
        io = _io_type(output, elementType)
        args = (cp, cb, codesOffset, sp, sb, scalesOffset, op, ob, outputOffset, _count(count),
                _stream_handle(stream, self.device))
        if keyBias is not None:
            if io != _lib.IO_F32:
                raise InvalidInput("key-bias removal takes float32 vectors")
            rc = self._lib.pitch_enqueue_decode_key_bias(ctypes.byref(config._c()), ctypes.byref(keyBias._c()), *args)
        elif io == _lib.IO_F32:
            rc = self._lib.pitch_enqueue_decode(ctypes.byref(config._c()), *args)
        else:
            rc = self._lib.pitch_enqueue_decode_io(ctypes.byref(config._c()), io, *args)
        _raise_for(rc)

    def enqueueDecodeBatch(self, items, config: QuantConfig, stream=None, elementType=None) -> None:
        """Decodes independent segments with one configuration in one call (pitch_enqueue_decode_batch), writing
        the same bytes as one enqueueDecode per segment. items: a sequence of (codes, scales, output, count) or
        (codes, scales, output, count, codesOffset, scalesOffset, outputOffset); every output has the element type
        elementType, else the first output's, chosen as for enqueueDecode. For a model's per-layer decodes
        (README.md:65-76 decodes each layer's cache with its own enqueueDecode); DecodeBatch keeps the segment
        table between calls."""
        items = list(items)
        if not items:
            raise InvalidInput("a batch needs at least one segment")
        io = _io_type(items[0][2], elementType)
        arr = (_lib.PitchDecodeItemC * len(items))()
        for i, it in enumerate(items):
            if len(it) not in (4, 7):
                raise InvalidInput("a segment is (codes, scales, output, count[, codesOffset, scalesOffset, "
                                   "outputOffset])")
            offs = it[4:] if len(it) == 7 else (0, 0, 0)
            _check_offsets(*offs)
            if _io_type(it[2], elementType) != io:
                raise InvalidInput("every segment's output must have the batch's element type")
            e = arr[i]
            e.codes, e.codes_bytes = _buf(it[0], "codes")
            e.scales, e.scales_bytes = _buf(it[1], "scales")
            e.output, e.output_bytes = _buf(it[2], "output")
            e.codes_offset, e.scales_offset, e.output_offset = (int(o) for o in offs)
            e.count = _count(it[3])
        _raise_for(self._lib.pitch_enqueue_decode_batch(ctypes.byref(config._c()), io, arr, len(items),
                                                        _stream_handle(stream, self.device)))

    def enqueuePerChannelAppend(self, input, codes, ranges, totalTokens: int, newTokens: int,
                                config: ChannelQuantConfig, inputOffset: int = 0, codesOffset: int = 0,
                                rangesOffset: int = 0, stream=None, elementType=None) -> None:
        """Appends newTokens to a head's per-channel cache of totalTokens - newTokens tokens, re-encoding the
        groups they touch (a growing partial group is re-encoded over all its tokens; README.md:85). input, codes
        and ranges are the head's whole buffers; the result equals one encode of all totalTokens tokens."""
        ip, ib = _buf(input, "input")
        cp, cb = _buf(codes, "codes")
        rp, rb = _buf(ranges, "ranges")
        _check_offsets(inputOffset, codesOffset, rangesOffset)
        rc = self._lib.pitch_enqueue_channel_append(ctypes.byref(config._c()), _io_type(input, elementType), ip, ib,
                                                    inputOffset, cp, cb, codesOffset, rp, rb, rangesOffset,
                                                    _count(totalTokens), _count(newTokens),
                                                    _stream_handle(stream, self.device))
        _raise_for(rc)

    # ---- attention over compressed caches (no counterpart in the reference; README.md:96)
    def enqueueAttentionDecode(self, q, keyCodes, keyScales, valueCodes, valueScales, output, tokens: int,
                               keyConfig: QuantConfig, valueConfig: QuantConfig | None = None, qPerKv: int = 1,
                               kvHeads: int = 1, tokenStride: int = 1, headStride: int | None = None,
                               scale: float | None = None, lse=None, workspace=None, stream=None,
                               noAlloc: bool = False, keyBias: KeyBias | None = None) -> None:
        """out = softmax(scale * q K^T) V over caches held as codes: q and output are fp32
        [kvHeads][qPerKv][dim]; the vector of (head h, token t) is t * tokenStride + h * headStride (default
        headStride = tokens, a head-major cache). scale defaults to 1 / sqrt(dim). lse, when given, receives the
        natural-log sum of exp of the scaled scores per query. Without a workspace one is allocated, unless
        noAlloc: then the call goes to pitch_enqueue_attention_decode_noalloc, which allocates nothing and uses the
        library's per-device scratch (at most PITCH_NOALLOC_SCRATCH_BYTES of workspace; per-vector keys only; calls
        overlapping on one device race).
        With a ChannelQuantConfig as keyConfig the keys are per-channel: keyScales is their fp16 ranges tensor, the
        caches are head-major (tokenStride 1) and headStride, in tokens, a multiple of the group size (default:
        tokens rounded up to it).
        With keyBias (per-vector keys encoded with that key bias, pitch_enqueue_attention_decode_key_bias) the
        scores use decode(k) + R_t b: keyBias.heads must be kvHeads and token t sits at keyBias.firstPosition + t."""
        torch = _torch()
        channel_keys = isinstance(keyConfig, ChannelQuantConfig)
        if channel_keys and valueConfig is None:
            raise InvalidInput("per-channel keys need a per-vector valueConfig")
        if keyBias is not None and (channel_keys or noAlloc):
            raise InvalidInput("key-bias removal takes per-vector keys and a workspace")
        valueConfig = valueConfig or keyConfig
        scale = 1.0 / math.sqrt(keyConfig.dim) if scale is None else scale
        if headStride is None:
            headStride = int(tokens) if not channel_keys else -(-int(tokens) // keyConfig.groupSize) * keyConfig.groupSize
        desc = _attention_desc(qPerKv, kvHeads, tokens, tokenStride, headStride, scale)
        if noAlloc and (channel_keys or workspace is not None):
            raise InvalidInput("noAlloc takes per-vector keys and no workspace")
        if workspace is None and not noAlloc:
            nbytes = attention_workspace_bytes(valueConfig if channel_keys else keyConfig, valueConfig, tokens,
                                               qPerKv, kvHeads)
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        args = []
        for t, name in ((q, "query"), (keyCodes, "key codes"), (keyScales, "key scales"), (valueCodes, "value codes"),
                        (valueScales, "value scales"), (output, "output")):
            p_, b_ = _buf(t, name)
            args += [p_, b_, 0]
        if lse is not None:
            p_, b_ = _buf(lse, "lse")
            args += [p_, b_, 0]
        else:
            args += [None, 0, 0]
        if noAlloc:
            rc = self._lib.pitch_enqueue_attention_decode_noalloc(
                ctypes.byref(keyConfig._c()), ctypes.byref(valueConfig._c()), ctypes.byref(desc), *args,
                _stream_handle(stream, self.device))
            _raise_for(rc)
            return
        wp, wb = _buf(workspace, "workspace")
        if keyBias is not None:
            rc = self._lib.pitch_enqueue_attention_decode_key_bias(
                ctypes.byref(keyConfig._c()), ctypes.byref(valueConfig._c()), ctypes.byref(desc),
                ctypes.byref(keyBias._c()), *args, wp, wb, _stream_handle(stream, self.device))
            _raise_for(rc)
            return
        fn = (self._lib.pitch_enqueue_attention_decode_channel_keys if channel_keys
              else self._lib.pitch_enqueue_attention_decode)
        rc = fn(ctypes.byref(keyConfig._c()), ctypes.byref(valueConfig._c()), ctypes.byref(desc), *args, wp, wb,
                _stream_handle(stream, self.device))
        _raise_for(rc)

    # ---- per-channel (PerChannel.swift:182-290)
    def encodePerChannel(self, vectors, dim: int | None = None, bits: int | None = None, groupSize: int = 64,
                         config: ChannelQuantConfig | None = None) -> ChannelCompressedBlock:
        torch = _torch()
        if config is None:
            config = ChannelQuantConfig(dim, bits, groupSize)
        n = int(vectors.numel()) if isinstance(vectors, torch.Tensor) else int(np.asarray(vectors).size)
        if n == 0 or n % config.dim != 0:
            raise InvalidInput(f"{n} floats is not a whole number of {config.dim}-dim tokens")
        _validate_values(vectors if isinstance(vectors, torch.Tensor) else np.asarray(vectors, dtype=np.float32),
                         ChannelQuantConfig.maxInputMagnitude, "per-channel ranges are stored in fp16")
        count = n // config.dim
        groups = config.groupCount(count)

        def run():
            x = self._on_device(vectors)
            codes = torch.empty(count * config.codeStride, dtype=torch.uint8, device=self.device)
            ranges = torch.empty(groups * config.rangeStride // 2, dtype=torch.int16, device=self.device)
            self.enqueuePerChannelEncode(x, codes, ranges, count, config)
            return codes, ranges

        codes, ranges = self._guard(run, EncodingFailed)
        return ChannelCompressedBlock(config, codes.cpu().numpy().tobytes(),
                                      ranges.cpu().numpy().view(np.uint16), _checked=False)

    def decodePerChannel(self, block: ChannelCompressedBlock) -> np.ndarray:
        torch = _torch()
        out = torch.empty(block.count * block.config.dim, dtype=torch.float32, device=self.device)
        self.decodePerChannel_into(block, out, 0)
        return out.cpu().numpy()

    def decodePerChannel_into(self, block: ChannelCompressedBlock, buffer, offset: int = 0) -> None:
        torch = _torch()
        block.validate()

        def run():
            codes = torch.from_numpy(np.frombuffer(block.codes, dtype=np.uint8).copy()).to(self.device)
            ranges = torch.from_numpy(block.ranges.view(np.int16).copy()).to(self.device)
            self.enqueuePerChannelDecode(codes, ranges, buffer, block.count, block.config, outputOffset=offset)

        self._guard(run, DecodingFailed)

    def enqueuePerChannelEncode(self, input, codes, ranges, count: int, config: ChannelQuantConfig,
                                inputOffset: int = 0, codesOffset: int = 0, rangesOffset: int = 0,
                                stream=None, elementType=None) -> None:
        ip, ib = _buf(input, "input")
        cp, cb = _buf(codes, "codes")
        rp, rb = _buf(ranges, "ranges")
        _check_offsets(inputOffset, codesOffset, rangesOffset)
        io = _io_type(input, elementType)
        args = (ip, ib, inputOffset, cp, cb, codesOffset, rp, rb, rangesOffset, _count(count),
                _stream_handle(stream, self.device))
        if io == _lib.IO_F32:
            rc = self._lib.pitch_enqueue_channel_encode(ctypes.byref(config._c()), *args)
        else:
            rc = self._lib.pitch_enqueue_channel_encode_io(ctypes.byref(config._c()), io, *args)
        _raise_for(rc)

    def enqueuePerChannelDecode(self, codes, ranges, output, count: int, config: ChannelQuantConfig,
                                codesOffset: int = 0, rangesOffset: int = 0, outputOffset: int = 0,
                                stream=None, elementType=None) -> None:
        cp, cb = _buf(codes, "codes")
        rp, rb = _buf(ranges, "ranges")
        op, ob = _buf(output, "output")
        _check_offsets(codesOffset, rangesOffset, outputOffset)
        io = _io_type(output, elementType)
        args = (cp, cb, codesOffset, rp, rb, rangesOffset, op, ob, outputOffset, _count(count),
                _stream_handle(stream, self.device))
        if io == _lib.IO_F32:
            rc = self._lib.pitch_enqueue_channel_decode(ctypes.byref(config._c()), *args)
        else:
            rc = self._lib.pitch_enqueue_channel_decode_io(ctypes.byref(config._c()), io, *args)
        _raise_for(rc)


class EncodeBatch:
    """A segment table for pitch_enqueue_encode_batch kept between calls: one segment per (input, codes, scales)
    buffer triple, e.g. one per layer's cache. Each enqueue sets the segments' counts and byte offsets in place
    (scalars or one value per segment) and issues one batched encode, so a decode step's append to every layer
    costs one call. The buffers are held for the table's lifetime."""

    def __init__(self, pitch: "PITCH", config: QuantConfig, inputs, codes, scales, elementType=None):
        self._pitch, self.config = pitch, config
        self._bufs = (list(inputs), list(codes), list(scales))
        n = len(self._bufs[0])
        if n < 1 or len(self._bufs[1]) != n or len(self._bufs[2]) != n:
            raise InvalidInput("inputs, codes and scales need one buffer per segment")
        self._io = _io_type(self._bufs[0][0], elementType)
        if any(_io_type(t, elementType) != self._io for t in self._bufs[0]):
            raise InvalidInput("every segment's input must have the batch's element type")
        self._arr = (_lib.PitchEncodeItemC * n)()
        self._tab = np.frombuffer(self._arr, dtype=np.uint64).reshape(n, 10)  # the C array's fields, in place
        for i in range(n):
            e = self._arr[i]
            e.input, e.input_bytes = _buf(self._bufs[0][i], "input")
            e.codes, e.codes_bytes = _buf(self._bufs[1][i], "codes")
            e.scales, e.scales_bytes = _buf(self._bufs[2][i], "scales")
        self._n = n

    def __len__(self) -> int:
        return self._n

    def enqueue(self, count, inputOffsets=0, codesOffsets=0, scalesOffsets=0, stream=None) -> None:
        for name, v in (("count", count), ("offset", inputOffsets), ("offset", codesOffsets),
                        ("offset", scalesOffsets)):
            a = np.asarray(v)
            if a.dtype.kind not in "iu" or (a < (1 if name == "count" else 0)).any():
                raise InvalidInput(f"{name} {v!r} must be {'at least 1' if name == 'count' else 'non-negative'}")
        t = self._tab
        t[:, 9] = count
        t[:, 2] = inputOffsets
        t[:, 5] = codesOffsets
        t[:, 8] = scalesOffsets
        p = self._pitch
        _raise_for(p._lib.pitch_enqueue_encode_batch(ctypes.byref(self.config._c()), self._io, self._arr, self._n,
                                                     _stream_handle(stream, p.device)))


class DecodeBatch:
    """A segment table for pitch_enqueue_decode_batch kept between calls: one segment per (codes, scales, output)
    buffer triple, e.g. one per layer's cache. Each enqueue sets the segments' counts and byte offsets in place
    (scalars or one value per segment) and issues one batched decode, so a decode step's per-layer decodes cost
    one call. The buffers are held for the table's lifetime."""

    def __init__(self, pitch: "PITCH", config: QuantConfig, codes, scales, outputs, elementType=None):
        self._pitch, self.config = pitch, config
        self._bufs = (list(codes), list(scales), list(outputs))
        n = len(self._bufs[0])
        if n < 1 or len(self._bufs[1]) != n or len(self._bufs[2]) != n:
            raise InvalidInput("codes, scales and outputs need one buffer per segment")
        self._io = _io_type(self._bufs[2][0], elementType)
        if any(_io_type(t, elementType) != self._io for t in self._bufs[2]):
            raise InvalidInput("every segment's output must have the batch's element type")
        self._arr = (_lib.PitchDecodeItemC * n)()
        self._tab = np.frombuffer(self._arr, dtype=np.uint64).reshape(n, 10)  # the C array's fields, in place
        for i in range(n):
            e = self._arr[i]
            e.codes, e.codes_bytes = _buf(self._bufs[0][i], "codes")
            e.scales, e.scales_bytes = _buf(self._bufs[1][i], "scales")
            e.output, e.output_bytes = _buf(self._bufs[2][i], "output")
        self._n = n

    def __len__(self) -> int:
        return self._n

    def enqueue(self, count, codesOffsets=0, scalesOffsets=0, outputOffsets=0, stream=None) -> None:
        for name, v in (("count", count), ("offset", codesOffsets), ("offset", scalesOffsets),
                        ("offset", outputOffsets)):
            a = np.asarray(v)
            if a.dtype.kind not in "iu" or (a < (1 if name == "count" else 0)).any():
                raise InvalidInput(f"{name} {v!r} must be {'at least 1' if name == 'count' else 'non-negative'}")
        t = self._tab
        t[:, 9] = count
        t[:, 2] = codesOffsets
        t[:, 5] = scalesOffsets
        t[:, 8] = outputOffsets
        p = self._pitch
        _raise_for(p._lib.pitch_enqueue_decode_batch(ctypes.byref(self.config._c()), self._io, self._arr, self._n,
                                                     _stream_handle(stream, p.device)))


def _attention_desc(q_per_kv: int, kv_heads: int, tokens: int, token_stride: int, head_stride: int,
                    scale: float) -> _lib.PitchAttentionDescC:
    for name, v in (("qPerKv", q_per_kv), ("kvHeads", kv_heads), ("tokens", tokens), ("tokenStride", token_stride),
                    ("headStride", head_stride)):
        if not isinstance(v, (int, np.integer)) or v < 0:
            raise InvalidInput(f"{name} {v} must be a non-negative integer")
    return _lib.PitchAttentionDescC(int(q_per_kv), int(kv_heads), int(tokens), int(token_stride), int(head_stride),
                                    float(scale), 0)


def attention_workspace_bytes(keyConfig: QuantConfig, valueConfig: QuantConfig, tokens: int, qPerKv: int = 1,
                              kvHeads: int = 1) -> int:
    """Device workspace pitch_enqueue_attention_decode needs for a call of this shape."""
    desc = _attention_desc(qPerKv, kvHeads, tokens, 1, tokens, 1.0)
    out = ctypes.c_uint64(0)
    _raise_for(_lib_or_raise().pitch_attention_workspace_size(ctypes.byref(keyConfig._c()),
                                                              ctypes.byref(valueConfig._c()), ctypes.byref(desc),
                                                              ctypes.byref(out)))
    return int(out.value)


def _check_offsets(*offs) -> None:
    for o in offs:
        if not isinstance(o, (int, np.integer)) or o < 0:
            raise InvalidInput(f"offset {o} must be a non-negative multiple of 4")


def _count(c) -> int:
    if not isinstance(c, (int, np.integer)) or c < 1:
        raise InvalidInput("count must be at least 1")
    return int(c)


# ----------------------------------------------------------------------------------------- function mirrors
# Function-level mirrors of reference/pitch_reference.py, on device tensors through the same kernels.
SUPPORTED_BITS = range(2, 9)
SUPPORTED_DIMS = [2 ** k for k in range(1, 11)]
CHANNEL_DEFAULT_GROUP = 64
FP16_MAX = 65504.0


def code_stride_bytes(d: int, b: int) -> int:
    """pitch_reference.py:65-66."""
    return ((d * b + 7) // 8 + 3) & ~3


def bits_per_coordinate(d: int, b: int) -> float:
    """pitch_reference.py:134-135."""
    return (code_stride_bytes(d, b) + 4) * 8 / d


def channel_group_count(n: int, G: int) -> int:
    return (n + G - 1) // G


def channel_bits_per_coordinate(d: int, b: int, G: int = CHANNEL_DEFAULT_GROUP) -> float:
    return code_stride_bytes(d, b) * 8 / d + 32 / G


def pack_codes(codes, b: int, stream=None):
    """(n, d) unpacked codes (integer tensor on the device) -> (n * codeStride,) uint8 packed codes."""
    torch = _torch()
    n, d = codes.shape
    u8 = codes.to(torch.uint8).contiguous()
    out = torch.empty(n * code_stride_bytes(d, b), dtype=torch.uint8, device=codes.device)
    up, ub = _buf(u8, "unpacked")
    pp, pb = _buf(out, "packed")
    with torch.cuda.device(codes.device):
        _raise_for(_lib_or_raise().pitch_enqueue_pack_codes(d, b, up, ub, 0, pp, pb, 0, n,
                                                            _stream_handle(stream, codes.device)))
    return out


def unpack_codes(packed, n: int, d: int, b: int, stream=None):
    """Packed codes (uint8 device tensor) -> (n, d) int64 codes."""
    torch = _torch()
    out = torch.empty(n * d, dtype=torch.uint8, device=packed.device)
    pp, pb = _buf(packed.contiguous(), "packed")
    up, ub = _buf(out, "unpacked")
    with torch.cuda.device(packed.device):
        _raise_for(_lib_or_raise().pitch_enqueue_unpack_codes(d, b, pp, pb, 0, up, ub, 0, n,
                                                              _stream_handle(stream, packed.device)))
    return out.view(n, d).to(torch.int64)


def _pitch_for(t) -> PITCH:
    return PITCH(device=t.device)


def _io_input(X):
    """X as a contiguous tensor the kernels read directly: float16 and bfloat16 stay 16-bit."""
    torch = _torch()
    return (X if X.dtype in (torch.float16, torch.bfloat16) else X.to(torch.float32)).contiguous()


def _encode_fn(method: str, X, b: int, seed: int):
    torch = _torch()
    n, d = X.shape
    cfg = QuantConfig(method, d, b, seed)
    x = _io_input(X)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=X.device)
    scales = torch.empty(n, dtype=torch.float32, device=X.device)
    with torch.cuda.device(X.device):
        _pitch_for(X).enqueueEncode(x, codes, scales, n, cfg)
    return unpack_codes(codes, n, d, b), scales


def _decode_fn(method: str, codes, scales, b: int, seed: int, dtype=None):
    torch = _torch()
    n, d = codes.shape
    cfg = QuantConfig(method, d, b, seed)
    packed = pack_codes(codes, b)
    out = torch.empty((n, d), dtype=dtype or torch.float32, device=codes.device)
    with torch.cuda.device(codes.device):
        _pitch_for(codes).enqueueDecode(packed, scales.to(torch.float32).contiguous(), out, n, cfg)
    return out


def turbo_encode(X, b: int, seed: int = DEFAULT_SEED):
    """(codes (n, d) int64, norms (n,) float32) (pitch_reference.py:92-102). X may be float16 or bfloat16: the
    kernels widen it to float32 exactly."""
    return _encode_fn("turboQuant", X, b, seed)


def turbo_decode(codes, norms, b: int, seed: int = DEFAULT_SEED, dtype=None):
    """pitch_reference.py:104-107; dtype float16 or bfloat16 rounds the float32 result to nearest even."""
    return _decode_fn("turboQuant", codes, norms, b, seed, dtype)


def polar_encode(X, b: int, seed: int = DEFAULT_SEED):
    """(codes (n, d) int64, rmax (n,) float32) (pitch_reference.py:109-121); X as for turbo_encode."""
    return _encode_fn("polarQuant", X, b, seed)


def polar_decode(codes, rmax, b: int, seed: int = DEFAULT_SEED, dtype=None):
    """pitch_reference.py:123-129; dtype as for turbo_decode."""
    return _decode_fn("polarQuant", codes, rmax, b, seed, dtype)


ENCODERS = {"turboQuant": turbo_encode, "polarQuant": polar_encode}
DECODERS = {"turboQuant": turbo_decode, "polarQuant": polar_decode}


def channel_encode(X, b: int, G: int = CHANNEL_DEFAULT_GROUP):
    """(codes (n, d) int64, ranges (groups, 2, d) float16) (pitch_reference.py:145-162); X may be float16 or
    bfloat16."""
    torch = _torch()
    n, d = X.shape
    cfg = ChannelQuantConfig(d, b, G)
    _validate_values(X, FP16_MAX, "per-channel ranges are stored in fp16")
    x = _io_input(X)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=X.device)
    ranges = torch.empty(cfg.groupCount(n) * 2 * d, dtype=torch.float16, device=X.device)
    with torch.cuda.device(X.device):
        _pitch_for(X).enqueuePerChannelEncode(x, codes, ranges, n, cfg)
    return unpack_codes(codes, n, d, b), ranges.view(cfg.groupCount(n), 2, d)


def channel_decode(codes, ranges, b: int, G: int = CHANNEL_DEFAULT_GROUP, dtype=None):
    """pitch_reference.py:165-174; dtype float16 or bfloat16 rounds the float32 result to nearest even."""
    torch = _torch()
    n, d = codes.shape
    cfg = ChannelQuantConfig(d, b, G)
    packed = pack_codes(codes, b)
    out = torch.empty((n, d), dtype=dtype or torch.float32, device=codes.device)
    with torch.cuda.device(codes.device):
        _pitch_for(codes).enqueuePerChannelDecode(packed, ranges.to(torch.float16).contiguous(), out, n, cfg)
    return out


def attention_decode(q, k_codes, k_scales, v_codes, v_scales, b: int, method: str = "turboQuant",
                     seed: int = DEFAULT_SEED, scale: float | None = None, v_bits: int | None = None,
                     v_method: str | None = None, v_seed: int | None = None):
    """Decode-step attention over compressed caches: q (kv_heads, q_per_kv, d) fp32, packed codes
    (kv_heads, T, codeStride) uint8 and scales (kv_heads, T) as the encoders write them, head-major. Returns
    (out (kv_heads, q_per_kv, d) fp32, lse (kv_heads, q_per_kv)), equal to softmax(scale q K^T) V over the
    decoded caches (reference/attention_extra.py:70-74) without writing them."""
    torch = _torch()
    if q.dim() == 2:
        q = q.unsqueeze(0)
    H, nq, d = q.shape
    T = k_codes.shape[1]
    kc = QuantConfig(method, d, b, seed)
    vc = QuantConfig(v_method or method, d, v_bits or b, seed if v_seed is None else v_seed)
    out = torch.empty((H, nq, d), dtype=torch.float32, device=q.device)
    lse = torch.empty((H, nq), dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _pitch_for(q).enqueueAttentionDecode(q.to(torch.float32).contiguous(), k_codes.contiguous(),
                                             k_scales.to(torch.float32).contiguous(), v_codes.contiguous(),
                                             v_scales.to(torch.float32).contiguous(), out, T, kc, vc, qPerKv=nq,
                                             kvHeads=H, tokenStride=1, headStride=T, scale=scale, lse=lse)
    return out, lse


def attention_decode_channel_keys(q, k_codes, k_ranges, v_codes, v_scales, k_bits: int, v_bits: int,
                                  group: int = CHANNEL_DEFAULT_GROUP, v_method: str = "turboQuant",
                                  v_seed: int = DEFAULT_SEED, scale: float | None = None):
    """attention_decode with per-channel keys: k_codes (kv_heads, T_pad, codeStride) uint8 and k_ranges
    (kv_heads, T_pad / group, 2, d) fp16 as per-head channel_encode calls write them, with T_pad the tokens
    rounded up to the group size; v_codes / v_scales per-vector over the same rows."""
    torch = _torch()
    if q.dim() == 2:
        q = q.unsqueeze(0)
    H, nq, d = q.shape
    T = k_codes.shape[1]
    kc = ChannelQuantConfig(d, k_bits, group)
    vc = QuantConfig(v_method, d, v_bits, v_seed)
    out = torch.empty((H, nq, d), dtype=torch.float32, device=q.device)
    lse = torch.empty((H, nq), dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _pitch_for(q).enqueueAttentionDecode(q.to(torch.float32).contiguous(), k_codes.contiguous(),
                                             k_ranges.contiguous(), v_codes.contiguous(),
                                             v_scales.to(torch.float32).contiguous(), out, T, kc, vc, qPerKv=nq,
                                             kvHeads=H, tokenStride=1, headStride=T, scale=scale, lse=lse)
    return out, lse


def rand_signs(seed: int, d: int):
    """+1 / -1 rotation signs (pitch_reference.py:17-19), host-side integer arithmetic as in the kernels."""
    i = (np.uint64(seed) + np.arange(d, dtype=np.uint64)) & np.uint64(0xFFFFFFFF)
    state = (i * np.uint64(747796405) + np.uint64(2891336453)) & np.uint64(0xFFFFFFFF)
    word = (((state >> ((state >> np.uint64(28)) + np.uint64(4))) ^ state) * np.uint64(277803737)) \
        & np.uint64(0xFFFFFFFF)
    h = ((word >> np.uint64(22)) ^ word) & np.uint64(0xFFFFFFFF)
    return np.where(h & np.uint64(1), 1.0, -1.0)

