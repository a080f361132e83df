/*
 * pitch_amd.h - C ABI of the MI355X (gfx950) KV-cache codec library libpitch_amd.so.
 *
 * Drop-in boundary for the codec path of SwiftCham/PITCH. Each entry point below replaces one operator of
 * the reference's Swift surface (file:line in /root/reference) with the same argument meaning, the same
 * validation and the same error categories. Buffers are device pointers owned by the caller; every offset
 * is in bytes and must be a non-negative multiple of 4; every length is the byte size of the whole buffer
 * starting at the pointer, so the library can perform the reference's "needs N bytes after offset" check.
 * The enqueue functions validate, launch on the given HIP stream and return without waiting, as the
 * reference's enqueue* calls encode into the caller's command buffer (Sources/PITCH/PITCH.swift:136-165).
 *
 * Deviation: counts and offsets are 64-bit, so a single call may cover count * dim >= 2^32 elements,
 * which the reference rejects (Sources/PITCH/Core/Codec.swift:30-32). Per-channel calls require
 * count < 2^32 tokens.
 */
#ifndef PITCH_AMD_H
#define PITCH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes, mirroring PITCHError (Sources/PITCH/Core/PITCHError.swift:10-19). */
#define PITCH_OK 0
#define PITCH_ERR_INVALID_INPUT (-1)          /* PITCHError.invalidInput */
#define PITCH_ERR_INVALID_BIT_WIDTH (-2)      /* PITCHError.invalidBitWidth */
#define PITCH_ERR_INVALID_DIMENSION (-3)      /* PITCHError.invalidDimension */
#define PITCH_ERR_CONFIGURATION_MISMATCH (-4) /* PITCHError.configurationMismatch */
#define PITCH_ERR_ENCODING_FAILED (-5)        /* PITCHError.encodingFailed */
#define PITCH_ERR_DECODING_FAILED (-6)        /* PITCHError.decodingFailed */
#define PITCH_ERR_DEVICE_UNAVAILABLE (-7)     /* PITCHError.metalNotSupported (no usable GPU) */

/* QuantMethod (Sources/PITCH/Models/QuantMethod.swift:8-11). */
#define PITCH_METHOD_TURBO 0u
#define PITCH_METHOD_POLAR 1u

/* Element type of the uncompressed vectors of the *_io entry points: what encode reads and decode writes.
 * The reference's codec is float32 only ("Inputs and outputs are float32; models that keep caches in fp16 or
 * bf16 need a conversion", README.md:97). 16-bit inputs are widened to float32 exactly and encoded as the
 * float32 entry point encodes them; decoded values are the float32 entry point's results rounded to nearest
 * even (overflow to infinity). Codes, scales and ranges are the same bytes for every element type. */
#define PITCH_IO_F32 0u
#define PITCH_IO_F16 1u
#define PITCH_IO_BF16 2u

/* Default rotation seed, PITCH.defaultSeed = 0x50495443 (Sources/PITCH/PITCH.swift:18). */
#define PITCH_DEFAULT_SEED 0x50495443u

/* QuantConfig (Sources/PITCH/Models/QuantConfig.swift:11-60); same 16-byte layout as BatchParams minus
 * count (Sources/PITCH/Core/Codec.swift:12-17). */
typedef struct pitch_config {
  uint32_t method; /* PITCH_METHOD_TURBO or PITCH_METHOD_POLAR */
  uint32_t dim;    /* power of two, 2..1024 */
  uint32_t bits;   /* 2..8 */
  uint32_t seed;   /* rotation seed */
} pitch_config_t;

/* ChannelQuantConfig (Sources/PITCH/PerChannel.swift:15-70). */
typedef struct pitch_channel_config {
  uint32_t dim;        /* channels per token, 1..1024 (any value) */
  uint32_t bits;       /* 2..8 */
  uint32_t group_size; /* tokens per group, 1..65536 */
  uint32_t reserved;   /* 0 */
} pitch_channel_config_t;

/* Library version as 0xMMmmpp. */
uint32_t pitch_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* pitch_last_error(void);

/* Validates and fills a QuantConfig; *code_stride = ceil(dim * bits / 32) * 4 bytes.
 * Replaces PITCH.config(method:dim:bits:) / QuantConfig.init (Sources/PITCH/PITCH.swift:53-55,
 * Sources/PITCH/Models/QuantConfig.swift:24-35,47). code_stride may be NULL. */
int pitch_config(uint32_t method, uint32_t dim, uint32_t bits, uint32_t seed, pitch_config_t* out,
                 uint32_t* code_stride);

/* Validates and fills a ChannelQuantConfig; *code_stride = ceil(dim * bits / 32) * 4 bytes and
 * *range_stride = 4 * dim bytes (fp16 minima then maxima per group).
 * Replaces PITCH.channelConfig(dim:bits:groupSize:) / ChannelQuantConfig.init
 * (Sources/PITCH/PerChannel.swift:184-187,30-43,55,58). Either output stride may be NULL. */
int pitch_channel_config(uint32_t dim, uint32_t bits, uint32_t group_size, pitch_channel_config_t* out,
                         uint32_t* code_stride, uint32_t* range_stride);

/* Encodes count contiguous fp32 vectors: writes count * code_stride bytes of packed codes and count fp32
 * scales (the norm for TurboQuant, the largest pair radius for PolarQuant).
 * Replaces PITCH.enqueueEncode(input:inputOffset:codes:codesOffset:scales:scalesOffset:count:config:
 * commandBuffer:) (Sources/PITCH/PITCH.swift:144-153 -> Sources/PITCH/Core/Codec.swift:70-103). */
int pitch_enqueue_encode(const pitch_config_t* config, const void* input, uint64_t input_bytes,
                         uint64_t input_offset, void* codes, uint64_t codes_bytes, uint64_t codes_offset,
                         void* scales, uint64_t scales_bytes, uint64_t scales_offset, uint64_t count,
                         void* stream /* hipStream_t; NULL = default stream */);

/* pitch_enqueue_encode with input elements of type io_type (PITCH_IO_*): the input buffer needs
 * count * dim * element-size bytes after its offset. Extends PITCH.enqueueEncode (Sources/PITCH/PITCH.swift:
 * 144-153) past its float32-only input (README.md:97). */
int pitch_enqueue_encode_io(const pitch_config_t* config, uint32_t io_type, const void* input,
                            uint64_t input_bytes, uint64_t input_offset, void* codes, uint64_t codes_bytes,
                            uint64_t codes_offset, void* scales, uint64_t scales_bytes, uint64_t scales_offset,
                            uint64_t count, void* stream);

/* One segment of a batched encode: count vectors of the batch's element type from input + input_offset, their
 * codes to codes + codes_offset and their scales to scales + scales_offset (byte offsets and sizes as in
 * pitch_enqueue_encode_io). */
typedef struct pitch_encode_item {
  const void* input;
  uint64_t input_bytes, input_offset;
  void* codes;
  uint64_t codes_bytes, codes_offset;
  void* scales;
  uint64_t scales_bytes, scales_offset;
  uint64_t count;
} pitch_encode_item_t;

/* Encodes n_items independent segments with one configuration and element type io_type (PITCH_IO_*) in as few
 * launches as it can (one per 32 segments), with the same codes and scales as one pitch_enqueue_encode_io per
 * segment. Every segment is validated as that call validates it, before anything is launched. For the
 * decode-phase append of a token's vectors across many layers: README.md:65-71 issues one
 * PITCH.enqueueEncode (Sources/PITCH/PITCH.swift:144-153) per cache, and a launch costs several microseconds
 * of host time here, so appending to 32 layers' caches through one call takes a fraction of 32 calls' time. */
int pitch_enqueue_encode_batch(const pitch_config_t* config, uint32_t io_type, const pitch_encode_item_t* items,
                               uint32_t n_items, void* stream);

/* Decodes count vectors into count * dim fp32 values. A vector's decoded bytes do not depend on the call: any count,
 * offset or batch that contains it writes the same bytes (every decode kernel runs the same arithmetic in the same
 * order; only the grid differs with the call's size).
 * Replaces PITCH.enqueueDecode(codes:codesOffset:scales:scalesOffset:output:outputOffset:count:config:
 * commandBuffer:) (Sources/PITCH/PITCH.swift:156-165 -> Sources/PITCH/Core/Codec.swift:107-140). */
int pitch_enqueue_decode(const pitch_config_t* config, const void* codes, uint64_t codes_bytes,
                         uint64_t codes_offset, const void* scales, uint64_t scales_bytes,
                         uint64_t scales_offset, void* output, uint64_t output_bytes, uint64_t output_offset,
                         uint64_t count, void* stream);

/* pitch_enqueue_decode writing elements of type io_type (PITCH_IO_*). Extends PITCH.enqueueDecode
 * (Sources/PITCH/PITCH.swift:156-165) past its float32-only output (README.md:97). */
int pitch_enqueue_decode_io(const pitch_config_t* config, uint32_t io_type, const void* codes,
                            uint64_t codes_bytes, uint64_t codes_offset, const void* scales, uint64_t scales_bytes,
                            uint64_t scales_offset, void* output, uint64_t output_bytes, uint64_t output_offset,
                            uint64_t count, void* stream);

/* One segment of a batched decode: count vectors' codes from codes + codes_offset and scales from scales +
 * scales_offset, decoded to output + output_offset (byte offsets and sizes as in pitch_enqueue_decode_io). */
typedef struct pitch_decode_item {
  const void* codes;
  uint64_t codes_bytes, codes_offset;
  const void* scales;
  uint64_t scales_bytes, scales_offset;
  void* output;
  uint64_t output_bytes, output_offset;
  uint64_t count;
} pitch_decode_item_t;

/* Decodes n_items independent segments with one configuration and output element type io_type (PITCH_IO_*) in as
 * few launches as it can (one per 32 segments of fewer than 2^18 vectors; a longer segment gets the launch of a
 * single call), writing the same bytes as one pitch_enqueue_decode_io per segment.
 * Every segment is validated as that call validates it, before anything is launched. For a model's per-layer
 * decodes (README.md:65-76 decodes each layer's cache with its own PITCH.enqueueDecode, Sources/PITCH/PITCH.swift:
 * 156-165): a layer of one decode step is a few tens of thousands of vectors, too few to fill the GPU alone, and
 * one call over every layer's cache runs at the rate of a bulk decode. */
int pitch_enqueue_decode_batch(const pitch_config_t* config, uint32_t io_type, const pitch_decode_item_t* items,
                               uint32_t n_items, void* stream);

/* Key-projection bias removal for the per-vector methods (reference/mechanism_eval.py:88-97,113-116: a model
 * whose key projection adds a bias b before RoPE has keys k = R_t W x + R_t b; compressing k - R_t b and adding
 * R_t b back restores the per-vector methods, README.md:28; "not yet built into the kernels", README.md:100).
 * Vector v of a call is token first_position + v / heads of head v % heads (a token-major [t][h] cache) and
 * carries o = b_h * cos_t + rotate_half(b_h) * sin_t, rotate_half(x) = (-x[dim/2:], x[:dim/2]), in float32 with
 * each product and the sum rounded once. All three tables are fp32 device memory. */
typedef struct pitch_key_bias {
  const void* bias;        /* [heads][dim]: the key projection's bias per KV head, before RoPE */
  uint64_t bias_bytes;
  const void* cos;         /* [positions][dim]: the model's RoPE cosines (rotate_half layout) */
  const void* sin;         /* [positions][dim]: the model's RoPE sines */
  uint64_t table_bytes;    /* bytes of cos and of sin each; positions = table_bytes / (4 * dim) */
  uint64_t first_position; /* position of the call's first token */
  uint32_t heads;          /* KV heads per token */
  uint32_t reserved;       /* 0 */
} pitch_key_bias_t;

/* pitch_enqueue_encode of x - o (fp32 input): the scales are the norms (or rmax) of the debiased keys. */
int pitch_enqueue_encode_key_bias(const pitch_config_t* config, const pitch_key_bias_t* key_bias, const void* input,
                                  uint64_t input_bytes, uint64_t input_offset, void* codes, uint64_t codes_bytes,
                                  uint64_t codes_offset, void* scales, uint64_t scales_bytes, uint64_t scales_offset,
                                  uint64_t count, void* stream);

/* pitch_enqueue_decode followed by + o (fp32 output). */
int pitch_enqueue_decode_key_bias(const pitch_config_t* config, const pitch_key_bias_t* key_bias, const void* codes,
                                  uint64_t codes_bytes, uint64_t codes_offset, const void* scales,
                                  uint64_t scales_bytes, uint64_t scales_offset, void* output, uint64_t output_bytes,
                                  uint64_t output_offset, uint64_t count, void* stream);

/* Encodes count tokens of one head's keys (token-major, dim channels) per channel over groups of
 * group_size tokens: writes count * code_stride bytes of codes and ceil(count / group_size) * range_stride
 * bytes of fp16 ranges laid out [group][min row of dim][max row of dim].
 * Replaces PITCH.enqueuePerChannelEncode(input:inputOffset:codes:codesOffset:ranges:rangesOffset:count:
 * config:commandBuffer:) (Sources/PITCH/PerChannel.swift:251-260 -> :338-363). */
int pitch_enqueue_channel_encode(const pitch_channel_config_t* config, const void* input,
                                 uint64_t input_bytes, uint64_t input_offset, void* codes,
                                 uint64_t codes_bytes, uint64_t codes_offset, void* ranges,
                                 uint64_t ranges_bytes, uint64_t ranges_offset, uint64_t count,
                                 void* stream);

/* pitch_enqueue_channel_encode with key elements of type io_type (PITCH_IO_*). Extends
 * PITCH.enqueuePerChannelEncode (Sources/PITCH/PerChannel.swift:251-260) past float32-only input
 * (README.md:97). */
int pitch_enqueue_channel_encode_io(const pitch_channel_config_t* config, uint32_t io_type, const void* input,
                                    uint64_t input_bytes, uint64_t input_offset, void* codes,
                                    uint64_t codes_bytes, uint64_t codes_offset, void* ranges,
                                    uint64_t ranges_bytes, uint64_t ranges_offset, uint64_t count,
                                    void* stream);

/* Decodes count per-channel tokens into count * dim fp32 values.
 * Replaces PITCH.enqueuePerChannelDecode(codes:codesOffset:ranges:rangesOffset:output:outputOffset:count:
 * config:commandBuffer:) (Sources/PITCH/PerChannel.swift:261-270 -> :365-389). */
int pitch_enqueue_channel_decode(const pitch_channel_config_t* config, const void* codes,
                                 uint64_t codes_bytes, uint64_t codes_offset, const void* ranges,
                                 uint64_t ranges_bytes, uint64_t ranges_offset, void* output,
                                 uint64_t output_bytes, uint64_t output_offset, uint64_t count,
                                 void* stream);

/* pitch_enqueue_channel_decode writing elements of type io_type (PITCH_IO_*). Extends
 * PITCH.enqueuePerChannelDecode (Sources/PITCH/PerChannel.swift:261-270) past float32-only output
 * (README.md:97). */
int pitch_enqueue_channel_decode_io(const pitch_channel_config_t* config, uint32_t io_type, const void* codes,
                                    uint64_t codes_bytes, uint64_t codes_offset, const void* ranges,
                                    uint64_t ranges_bytes, uint64_t ranges_offset, void* output,
                                    uint64_t output_bytes, uint64_t output_offset, uint64_t count,
                                    void* stream);

/* Appends new_tokens tokens to one head's per-channel cache that already holds total_tokens - new_tokens of
 * them, re-encoding every group the new tokens touch: a partial last group is encoded again over all of its
 * tokens, so its fp16 ranges always cover the tokens it holds ("the newest, partial group can be kept in full
 * precision or re-encoded as it grows", README.md:85; the reference's ChannelCompressedBlock.append refuses
 * to append after a partial group, Sources/PITCH/PerChannel.swift:120-130). input holds the head's keys of
 * tokens [0, total_tokens) in the element type io_type (only the touched groups are read); codes and ranges
 * are the head's whole cache buffers, laid out as pitch_enqueue_channel_encode writes them. The result is
 * byte for byte that of one pitch_enqueue_channel_encode_io over all total_tokens tokens. */
int pitch_enqueue_channel_append(const pitch_channel_config_t* config, uint32_t io_type, const void* input,
                                 uint64_t input_bytes, uint64_t input_offset, void* codes, uint64_t codes_bytes,
                                 uint64_t codes_offset, void* ranges, uint64_t ranges_bytes, uint64_t ranges_offset,
                                 uint64_t total_tokens, uint64_t new_tokens, void* stream);

/* Decode-phase attention over compressed caches (no counterpart in the reference: it evaluates attention on
 * decoded caches, reference/attention_extra.py:70-74, and names decoding inside attention as its next step,
 * README.md:96). For each of kv_heads KV heads and each of its q_per_kv query heads:
 *   out = softmax(scale * q . K^T) V,  lse = log sum exp(scale * q . K^T)  (natural log)
 * where K and V are the decodes of the per-vector codes (TurboQuant or PolarQuant, any bit width 2..8, key and
 * value configs may differ in method, bits and seed but not in dimension, which must be 64 or 128). The codes
 * are read as stored; no decoded vector is written. Queries and outputs are fp32 [kv_heads][q_per_kv][dim].
 * The cache vector of (KV head h, token t) is t * token_stride + h * head_stride, in units of vectors, for
 * both the codes (code_stride bytes each) and the scales (4 bytes each): a token-major [t][h] cache has
 * token_stride = number of heads and head_stride = 1; a head-major [h][t] one has token_stride = 1. */
typedef struct pitch_attention_desc {
  uint32_t q_per_kv;     /* query heads per KV head (grouped-query attention), 1..8 */
  uint32_t kv_heads;     /* KV heads in the call, 1..65535 */
  uint64_t tokens;       /* cached tokens per KV head, >= 1 */
  uint64_t token_stride; /* vectors between consecutive tokens of one head */
  uint64_t head_stride;  /* vectors between consecutive KV heads */
  float scale;           /* softmax scale applied to q . k, e.g. 1 / sqrt(dim) */
  uint32_t reserved;     /* 0 */
} pitch_attention_desc_t;

/* Bytes of device workspace pitch_enqueue_attention_decode needs for these arguments. */
int pitch_attention_workspace_size(const pitch_config_t* key_config, const pitch_config_t* value_config,
                                   const pitch_attention_desc_t* desc, uint64_t* bytes);

/* Enqueues the attention described above on the stream. lse may be NULL. The workspace (at least
 * pitch_attention_workspace_size bytes of device memory) must not be used by another call until this one has
 * completed on the stream. */
int pitch_enqueue_attention_decode(const pitch_config_t* key_config, const pitch_config_t* value_config,
                                   const pitch_attention_desc_t* desc, const void* q, uint64_t q_bytes,
                                   uint64_t q_offset, const void* key_codes, uint64_t key_codes_bytes,
                                   uint64_t key_codes_offset, const void* key_scales, uint64_t key_scales_bytes,
                                   uint64_t key_scales_offset, const void* value_codes, uint64_t value_codes_bytes,
                                   uint64_t value_codes_offset, const void* value_scales,
                                   uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output,
                                   uint64_t output_bytes, uint64_t output_offset, void* lse, uint64_t lse_bytes,
                                   uint64_t lse_offset, void* workspace, uint64_t workspace_bytes, void* stream);

/* pitch_enqueue_attention_decode over a key cache encoded with key-bias removal (pitch_enqueue_encode_key_bias):
 * the scores are q . (decode(k) + o_t) with o_t = b_h cos_t + rotate_half(b_h) sin_t, the cache's k - o_t
 * restored as pitch_enqueue_decode_key_bias restores it (reference/mechanism_eval.py:113-116: the keys are
 * compress(k - R_t b) + R_t b). key_bias->heads must equal desc->kv_heads (row h of the bias is KV head h) and
 * token t of the cache is at position key_bias->first_position + t, so the tables need first_position + tokens
 * rows. Per-vector keys only (per-channel keys need no bias removal). Extends the fused attention, which the
 * reference does not have (README.md:96, 100). */
int pitch_enqueue_attention_decode_key_bias(
    const pitch_config_t* key_config, const pitch_config_t* value_config, const pitch_attention_desc_t* desc,
    const pitch_key_bias_t* key_bias, const void* q, uint64_t q_bytes, uint64_t q_offset, const void* key_codes,
    uint64_t key_codes_bytes, uint64_t key_codes_offset, const void* key_scales, uint64_t key_scales_bytes,
    uint64_t key_scales_offset, const void* value_codes, uint64_t value_codes_bytes, uint64_t value_codes_offset,
    const void* value_scales, uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output,
    uint64_t output_bytes, uint64_t output_offset, void* lse, uint64_t lse_bytes, uint64_t lse_offset,
    void* workspace, uint64_t workspace_bytes, void* stream);

/* Largest workspace pitch_enqueue_attention_decode_noalloc can serve, in bytes (32 MiB: e.g. 8 KV heads x 4 query
 * heads x 131072 tokens at dim 128 needs 18.9 MB). */
#define PITCH_NOALLOC_SCRATCH_BYTES (32ull << 20)

/* pitch_enqueue_attention_decode without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart in
 * the reference. The workspace is a scratch array compiled into the library, one per device, held until the process
 * ends; the call allocates nothing. Calls whose workspace (pitch_attention_workspace_size) exceeds
 * PITCH_NOALLOC_SCRATCH_BYTES fail with PITCH_ERR_INVALID_INPUT before any work is issued. Every call on a device
 * shares that device's array: calls that overlap on one device (on different streams, or from different threads
 * without ordering) race and must not be issued; calls ordered on one stream are safe. Results are otherwise those
 * of pitch_enqueue_attention_decode on the same arguments. The array's device address is looked up (one
 * hipGetSymbolAddress, no allocation) by the first call of any pitch_enqueue_* entry point on the device, so a caller
 * that captures a HIP graph makes that lookup outside the capture by issuing any one call on the device first. */
int pitch_enqueue_attention_decode_noalloc(const pitch_config_t* key_config, const pitch_config_t* value_config,
                                           const pitch_attention_desc_t* desc, const void* q, uint64_t q_bytes,
                                           uint64_t q_offset, const void* key_codes, uint64_t key_codes_bytes,
                                           uint64_t key_codes_offset, const void* key_scales,
                                           uint64_t key_scales_bytes, uint64_t key_scales_offset,
                                           const void* value_codes, uint64_t value_codes_bytes,
                                           uint64_t value_codes_offset, const void* value_scales,
                                           uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output,
                                           uint64_t output_bytes, uint64_t output_offset, void* lse,
                                           uint64_t lse_bytes, uint64_t lse_offset, void* stream);

/* pitch_enqueue_attention_decode with per-channel (KIVI) keys and per-vector values: the configuration the
 * reference recommends for models whose key projection has a bias (README.md:30) and evaluates as
 * "kivi_K{b}_turboV{b}" (reference/attention_extra.py:57-59). Keys decode as f32(c) * step + lo per group and
 * channel (reference/pitch_reference.py:165-174). The key cache is head-major, as per-head
 * pitch_enqueue_channel_encode calls write it: codes of (head h, token t) at row h * head_stride + t, fp16 ranges
 * of (h, group g) at group h * head_stride / group_size + g; desc->token_stride must be 1 and, with more than one
 * KV head, head_stride a multiple of the group size holding the tokens (one head: head_stride is ignored). The
 * values use the same rows. The group size must be a multiple of 64. */
int pitch_attention_channel_keys_workspace_size(const pitch_channel_config_t* key_config,
                                                const pitch_config_t* value_config, const pitch_attention_desc_t* desc,
                                                uint64_t* bytes);
int pitch_enqueue_attention_decode_channel_keys(
    const pitch_channel_config_t* key_config, const pitch_config_t* value_config, const pitch_attention_desc_t* desc,
    const void* q, uint64_t q_bytes, uint64_t q_offset, const void* key_codes, uint64_t key_codes_bytes,
    uint64_t key_codes_offset, const void* key_ranges, uint64_t key_ranges_bytes, uint64_t key_ranges_offset,
    const void* value_codes, uint64_t value_codes_bytes, uint64_t value_codes_offset, const void* value_scales,
    uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output, uint64_t output_bytes,
    uint64_t output_offset, void* lse, uint64_t lse_bytes, uint64_t lse_offset, void* workspace,
    uint64_t workspace_bytes, void* stream);

/* Packs count rows of dim unpacked codes (one uint8 per code, each < 2^bits) into count * code_stride
 * bytes, code i at bits [i * bits, i * bits + bits) of the row's little-endian 32-bit words.
 * Replaces pack_codes (reference/pitch_reference.py:68-78). */
int pitch_enqueue_pack_codes(uint32_t dim, uint32_t bits, const void* unpacked, uint64_t unpacked_bytes,
                             uint64_t unpacked_offset, void* packed, uint64_t packed_bytes,
                             uint64_t packed_offset, uint64_t count, void* stream);

/* Inverse of pitch_enqueue_pack_codes. Replaces unpack_codes (reference/pitch_reference.py:80-90). */
int pitch_enqueue_unpack_codes(uint32_t dim, uint32_t bits, const void* packed, uint64_t packed_bytes,
                               uint64_t packed_offset, void* unpacked, uint64_t unpacked_bytes,
                               uint64_t unpacked_offset, uint64_t count, void* stream);

/* Self-test of a hardware property the per-channel encoder relies on; no counterpart in the reference. The
 * encoder forms the correctly rounded reciprocal of each channel's step as v_rcp_f32 plus one Newton step,
 * which on gfx950 equals the correctly rounded 1 / x for every positive normal float below 2^126. This call
 * checks all of them on the current device (synchronously, allocating 4 MB of device memory) and writes
 * the number that differ (0 expected) to *mismatches. For tests and bring-up on new hardware. */
int pitch_selftest_reciprocal(uint64_t* mismatches);

#ifdef __cplusplus
}
#endif

#endif /* PITCH_AMD_H */
