"""pitch_amd: the MI355X (gfx950) KV-cache codec of SwiftCham/PITCH, as hand-written HIP kernels behind a C ABI.

The operator surface mirrors the reference: ``PITCH`` (config / encode / decode / enqueueEncode /
enqueueDecode and the per-channel forms), ``QuantConfig``, ``ChannelQuantConfig``, ``CompressedBatch``,
``ChannelCompressedBlock``, the ``PITCHError`` family, and function-level mirrors of
reference/pitch_reference.py (``turbo_encode``, ``polar_decode``, ``channel_encode``, ``pack_codes``, ...)
that run on device tensors. ``PITCH.enqueueEncodeBatch`` / ``EncodeBatch`` encode many caches' segments (a
token's append to every layer) in one call, and ``PITCH.enqueueDecodeBatch`` / ``DecodeBatch`` decode them. ``attention_decode`` / ``PITCH.enqueueAttentionDecode`` compute decode-step
attention directly over the compressed caches.
"""
from .api import (  # noqa: F401
    CHANNEL_DEFAULT_GROUP, DECODERS, DEFAULT_SEED, ENCODERS, FP16_MAX, PITCH, SUPPORTED_BITS, SUPPORTED_DIMS,
    ChannelCompressedBlock, ChannelQuantConfig, CompressedBatch, ConfigurationMismatch, DecodeBatch, DecodingFailed,
    DeviceUnavailable, EncodeBatch, EncodingFailed, InvalidBitWidth, InvalidDimension, InvalidInput, KeyBias, PITCHError,
    QuantConfig, QuantMethod, attention_decode, attention_decode_channel_keys, attention_workspace_bytes, bits_per_coordinate, channel_bits_per_coordinate, channel_decode, channel_encode,
    channel_group_count, code_stride_bytes, half_to_float, pack_codes, polar_decode, polar_encode, rand_signs,
    turbo_decode, turbo_encode, unpack_codes,
)

__version__ = "0.1.0"
