"""ctypes binding of libpitch_amd.so (the C ABI in include/pitch_amd.h).

There is no fallback: if the library is missing or fails to load, every codec call raises
DeviceUnavailable with the reason.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpitch_amd.so"

PITCH_OK = 0
ERR_INVALID_INPUT = -1
ERR_INVALID_BIT_WIDTH = -2
ERR_INVALID_DIMENSION = -3
ERR_CONFIGURATION_MISMATCH = -4
ERR_ENCODING_FAILED = -5
ERR_DECODING_FAILED = -6
ERR_DEVICE_UNAVAILABLE = -7

NOALLOC_SCRATCH_BYTES = 32 << 20   # PITCH_NOALLOC_SCRATCH_BYTES: workspace limit of the allocation-free attention

IO_F32 = 0    # element types of uncompressed vectors (PITCH_IO_*)
IO_F16 = 1
IO_BF16 = 2


class PitchConfigC(ctypes.Structure):
    _fields_ = [("method", ctypes.c_uint32), ("dim", ctypes.c_uint32), ("bits", ctypes.c_uint32),
                ("seed", ctypes.c_uint32)]


class PitchAttentionDescC(ctypes.Structure):
    _fields_ = [("q_per_kv", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("tokens", ctypes.c_uint64),
                ("token_stride", ctypes.c_uint64), ("head_stride", ctypes.c_uint64), ("scale", ctypes.c_float),
                ("reserved", ctypes.c_uint32)]


class PitchKeyBiasC(ctypes.Structure):
    _fields_ = [("bias", ctypes.c_void_p), ("bias_bytes", ctypes.c_uint64), ("cos", ctypes.c_void_p),
                ("sin", ctypes.c_void_p), ("table_bytes", ctypes.c_uint64), ("first_position", ctypes.c_uint64),
                ("heads", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class PitchEncodeItemC(ctypes.Structure):
    """pitch_encode_item_t: one segment of pitch_enqueue_encode_batch (ten 64-bit fields)."""
    _fields_ = [("input", ctypes.c_void_p), ("input_bytes", ctypes.c_uint64), ("input_offset", ctypes.c_uint64),
                ("codes", ctypes.c_void_p), ("codes_bytes", ctypes.c_uint64), ("codes_offset", ctypes.c_uint64),
                ("scales", ctypes.c_void_p), ("scales_bytes", ctypes.c_uint64), ("scales_offset", ctypes.c_uint64),
                ("count", ctypes.c_uint64)]


class PitchDecodeItemC(ctypes.Structure):
    """pitch_decode_item_t: one segment of pitch_enqueue_decode_batch (ten 64-bit fields)."""
    _fields_ = [("codes", ctypes.c_void_p), ("codes_bytes", ctypes.c_uint64), ("codes_offset", ctypes.c_uint64),
                ("scales", ctypes.c_void_p), ("scales_bytes", ctypes.c_uint64), ("scales_offset", ctypes.c_uint64),
                ("output", ctypes.c_void_p), ("output_bytes", ctypes.c_uint64), ("output_offset", ctypes.c_uint64),
                ("count", ctypes.c_uint64)]


class PitchChannelConfigC(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_uint32), ("bits", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32)]


_u32, _u64, _vp, _int = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int

# name -> (restype, argtypes); every symbol declared in include/pitch_amd.h
SIGNATURES = {
    "pitch_version": (_u32, []),
    "pitch_last_error": (ctypes.c_char_p, []),
    "pitch_config": (_int, [_u32, _u32, _u32, _u32, ctypes.POINTER(PitchConfigC), ctypes.POINTER(_u32)]),
    "pitch_channel_config": (_int, [_u32, _u32, _u32, ctypes.POINTER(PitchChannelConfigC),
                                    ctypes.POINTER(_u32), ctypes.POINTER(_u32)]),
    "pitch_enqueue_encode": (_int, [ctypes.POINTER(PitchConfigC), _vp, _u64, _u64, _vp, _u64, _u64,
                                    _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_decode": (_int, [ctypes.POINTER(PitchConfigC), _vp, _u64, _u64, _vp, _u64, _u64,
                                    _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_channel_encode": (_int, [ctypes.POINTER(PitchChannelConfigC), _vp, _u64, _u64, _vp,
                                            _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_channel_decode": (_int, [ctypes.POINTER(PitchChannelConfigC), _vp, _u64, _u64, _vp,
                                            _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_encode_io": (_int, [ctypes.POINTER(PitchConfigC), _u32, _vp, _u64, _u64, _vp, _u64, _u64,
                                       _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_encode_batch": (_int, [ctypes.POINTER(PitchConfigC), _u32, ctypes.POINTER(PitchEncodeItemC),
                                          _u32, _vp]),
    "pitch_enqueue_decode_batch": (_int, [ctypes.POINTER(PitchConfigC), _u32, ctypes.POINTER(PitchDecodeItemC),
                                          _u32, _vp]),
    "pitch_enqueue_decode_io": (_int, [ctypes.POINTER(PitchConfigC), _u32, _vp, _u64, _u64, _vp, _u64, _u64,
                                       _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_channel_encode_io": (_int, [ctypes.POINTER(PitchChannelConfigC), _u32, _vp, _u64, _u64, _vp,
                                               _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_channel_decode_io": (_int, [ctypes.POINTER(PitchChannelConfigC), _u32, _vp, _u64, _u64, _vp,
                                               _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_encode_key_bias": (_int, [ctypes.POINTER(PitchConfigC), ctypes.POINTER(PitchKeyBiasC), _vp, _u64,
                                             _u64, _vp, _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_decode_key_bias": (_int, [ctypes.POINTER(PitchConfigC), ctypes.POINTER(PitchKeyBiasC), _vp, _u64,
                                             _u64, _vp, _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_channel_append": (_int, [ctypes.POINTER(PitchChannelConfigC), _u32, _vp, _u64, _u64, _vp, _u64,
                                            _u64, _vp, _u64, _u64, _u64, _u64, _vp]),
    "pitch_attention_workspace_size": (_int, [ctypes.POINTER(PitchConfigC), ctypes.POINTER(PitchConfigC),
                                              ctypes.POINTER(PitchAttentionDescC), ctypes.POINTER(_u64)]),
    "pitch_enqueue_attention_decode": (_int, [ctypes.POINTER(PitchConfigC), ctypes.POINTER(PitchConfigC),
                                              ctypes.POINTER(PitchAttentionDescC)] + [_vp, _u64, _u64] * 7
                                       + [_vp, _u64, _vp]),
    "pitch_enqueue_attention_decode_key_bias": (_int, [ctypes.POINTER(PitchConfigC), ctypes.POINTER(PitchConfigC),
                                                       ctypes.POINTER(PitchAttentionDescC),
                                                       ctypes.POINTER(PitchKeyBiasC)] + [_vp, _u64, _u64] * 7
                                                + [_vp, _u64, _vp]),
    "pitch_enqueue_attention_decode_noalloc": (_int, [ctypes.POINTER(PitchConfigC), ctypes.POINTER(PitchConfigC),
                                                      ctypes.POINTER(PitchAttentionDescC)] + [_vp, _u64, _u64] * 7
                                               + [_vp]),
    "pitch_attention_channel_keys_workspace_size": (_int, [ctypes.POINTER(PitchChannelConfigC),
                                                           ctypes.POINTER(PitchConfigC),
                                                           ctypes.POINTER(PitchAttentionDescC), ctypes.POINTER(_u64)]),
    "pitch_enqueue_attention_decode_channel_keys": (_int, [ctypes.POINTER(PitchChannelConfigC),
                                                           ctypes.POINTER(PitchConfigC),
                                                           ctypes.POINTER(PitchAttentionDescC)] + [_vp, _u64, _u64] * 7
                                                    + [_vp, _u64, _vp]),
    "pitch_enqueue_pack_codes": (_int, [_u32, _u32, _vp, _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_enqueue_unpack_codes": (_int, [_u32, _u32, _vp, _u64, _u64, _vp, _u64, _u64, _u64, _vp]),
    "pitch_selftest_reciprocal": (_int, [ctypes.POINTER(_u64)]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def load() -> ctypes.CDLL:
    """Loads the library once; raises RuntimeError with the reason if it cannot."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                _load_error = (f"HIP extension {LIB_PATH.name} is not built (expected at {LIB_PATH}); "
                               "run `python -m pitch_amd.build`")
                raise RuntimeError(_load_error)
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    return load().pitch_last_error().decode("utf-8", "replace")
