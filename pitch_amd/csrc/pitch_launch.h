// Internal launch interface between the C ABI (pitch_abi.cpp) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Launch-shape tuning macros (compile-time; the library reads no environment variables).
#ifndef PITCH_ATTN_CHUNK
#define PITCH_ATTN_CHUNK 0  // attention tokens per chunk: 0 = by call size (attention_chunk_tokens)
#endif
#ifndef PITCH_ATTN_MIN_WG
#define PITCH_ATTN_MIN_WG 512  // attention_chunk_tokens halves the chunk until the call has this many workgroups
#endif
#ifndef PITCH_SLICE_ROUNDS
#define PITCH_SLICE_ROUNDS -1  // rounds per launch of every sliced call: -1 = each kernel's own default
#endif
#ifndef PITCH_STREAM_MIN_VECTORS
#define PITCH_STREAM_MIN_VECTORS (1u << 19)  // smallest float32 D = 1024 decode run by the streaming decoder
#endif
#ifndef PITCH_BLOCKS_PER_CU
#define PITCH_BLOCKS_PER_CU 0  // resident 256-thread blocks per CU of persistent grids: 0 = occupancy
#endif
#ifndef PITCH_ENC_BLOCKS_PER_WG
#define PITCH_ENC_BLOCKS_PER_WG 8  // blocks per workgroup of long staged encodes: 0 = always persistent
#endif
#ifndef PITCH_ENC_MIN_ROUNDS
// resident rounds from which a staged encode is oversubscribed. With the persistent launch's fair wave priority
// the persistent grid won at 32 and 48 rounds (d = 64: +3 points) and the oversubscribed one from 64 rounds up
// (d = 64 and 128: +1-5 points), equal at 56 (d = 128)
#define PITCH_ENC_MIN_ROUNDS 56
#endif

namespace pitch {

// Arguments of one per-vector encode or decode launch (pointers already advanced by the byte offsets).
struct VecArgs {
  const void* in;            // encode: count * dim elements of the I/O type
  const uint32_t* codes_in;  // decode: count * code_stride bytes
  uint32_t* codes_out;       // encode
  const float* scales_in;    // decode: count fp32
  float* scales_out;         // encode
  void* out;                 // decode: count * dim elements of the I/O type
  uint64_t count;
  uint32_t seed;
  uint32_t kb_heads;         // key-bias removal: heads per token (0 = no bias)
  // Key-bias removal (null kb_bias = none): vector v is token kb_first + v / kb_heads of head v % kb_heads and
  // carries the offset o = b * cos_t + rotate_half(b) * sin_t; encode takes x - o, decode writes x + o.
  const float* kb_bias;      // [heads][dim]
  const float* kb_cos;       // [positions][dim]
  const float* kb_sin;       // [positions][dim]
  uint64_t kb_first;
  // Rotation signs per team lane: bit e of lane_flips[t] is 1 when the coordinate held as element e by
  // team lane t has sign -1 (filled by the launcher from the seed).
  uint32_t lane_flips[32];
  // Encoders: 1 when the launch is persistent (every wave keeps one fixed share of the blocks) and the shares are
  // more than one block; the staged, transposed and lane-per-vector encoders then order their waves by the share
  // still to do (FairPriority).
  uint32_t fair;
};

// Arguments of one batched encode launch: up to kBatchItems independent segments with one configuration.
// Segment i (count[i] vectors from in[i] to codes_out[i] / scales_out[i]) is encoded by the workgroups
// [block_start[i], block_start[i + 1]); block_start[items] is the grid size (the launcher fills block_start).
// common supplies the seed (the launcher fills its lane_flips); its pointers and count are unused.
constexpr uint32_t kBatchItems = 32;
struct VecBatchArgs {
  VecArgs common;
  uint32_t items;
  uint32_t block_start[kBatchItems + 1];
  const void* in[kBatchItems];
  uint32_t* codes_out[kBatchItems];
  float* scales_out[kBatchItems];
  uint64_t count[kBatchItems];
};

// Arguments of one batched decode launch: up to kBatchItems independent segments with one configuration. Segment i
// (count[i] vectors from codes_in[i] / scales_in[i] to out[i]) is decoded by the workgroups [block_start[i],
// block_start[i + 1]) (the launcher fills block_start); common supplies the seed (the launcher fills its
// lane_flips).
struct DecBatchArgs {
  VecArgs common;
  uint32_t items;
  uint32_t block_start[kBatchItems + 1];
  const uint32_t* codes_in[kBatchItems];
  const float* scales_in[kBatchItems];
  void* out[kBatchItems];
  uint64_t count[kBatchItems];
};

// Arguments of one per-channel (KIVI) launch.
struct ChanArgs {
  const void* in;   // encode: count * dim elements of the I/O type
  const uint32_t* codes_in;
  uint32_t* codes_out;
  const uint16_t* ranges_in;  // fp16 bits, [group][min row][max row]
  uint16_t* ranges_out;
  void* out;        // decode: count * dim elements of the I/O type
  uint32_t count;   // tokens
  uint32_t dim;     // channels
  uint32_t group;   // tokens per group
  uint32_t nwords;  // 32-bit words of codes per token
};

// Arguments of a generic pack / unpack launch (unpacked codes are one byte each).
struct PackArgs {
  const uint8_t* unpacked_in;
  uint8_t* unpacked_out;
  const uint32_t* packed_in;
  uint32_t* packed_out;
  uint64_t count;
  uint32_t dim;
  uint32_t bits;
};

// Arguments of one decode-phase attention launch over compressed K and V caches (see pitch_attention.hip).
// Vector index of (KV head h, token t) in both caches: t * token_stride + h * head_stride.
struct AttnArgs {
  const float* q;            // [kv_heads][nq][dim] fp32 queries
  const uint32_t* k_codes;   // per-vector codes of the keys
  const float* k_scales;     // key norms (TurboQuant) or rmax (PolarQuant)
  const uint32_t* v_codes;
  const float* v_scales;
  float* out;                // [kv_heads][nq][dim] fp32
  float* lse;                // [kv_heads][nq] natural-log sum of exp of the scaled scores, or null
  float* ws;                 // workspace (attention_workspace_floats floats)
  uint64_t tokens;           // cached tokens per KV head
  uint64_t token_stride;
  uint64_t head_stride;
  uint32_t dim, nq, nqp;     // head dim; query heads per KV head; nq rounded up to 1, 2, 4 or 8
  uint32_t kv_heads;
  uint32_t kbits, vbits, kpolar, vpolar, kseed, vseed;
  uint32_t chunk, chunks;    // tokens per workgroup and chunks per KV head
  float qscale;              // softmax scale * log2(e) / sqrt(dim), folded into the rotated queries
  float oscale;              // 1 / sqrt(dim) of the value decode
  // Per-channel (KIVI) keys instead of per-vector ones (k_ranges non-null): codes [h][token] at
  // (t + h * head_stride) rows, fp16 ranges [h][group][2][dim] with head_stride / k_group groups per head.
  const uint16_t* k_ranges;
  uint32_t k_group;          // tokens per key group (a multiple of 64)
  float kscale;              // softmax scale * log2(e), folded into the per-group query products
  // Key-bias removal (kb_cos non-null, per-vector keys): the keys were encoded as k - o_t with
  // o_t = b_h cos_t + rotate_half(b_h) sin_t at position kb_first + t, and the scores add q . o_t.
  const float* kb_bias;      // [kv_heads][dim]
  const float* kb_cos;       // [positions][dim]
  const float* kb_sin;       // [positions][dim]
  uint64_t kb_first;
};

// Chunk length (tokens per workgroup) the attention kernels use for a call, and the workspace it needs.
uint32_t attention_chunk_tokens(uint64_t tokens, uint32_t kv_heads);
uint64_t attention_workspace_floats(uint32_t dim, uint32_t nqp, uint32_t kv_heads, uint64_t tokens, uint32_t chunk);
hipError_t launch_attention_d64(const AttnArgs& a, hipStream_t s);
hipError_t launch_attention_d128(const AttnArgs& a, hipStream_t s);

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Grid size for a grid-stride kernel: enough workgroups to fill every CU at the kernel's occupancy,
// but no more than the work needs. With balance_rounds, a call of several rounds may use fewer workgroups per
// CU so that its last round is not left nearly empty (for bandwidth-bound kernels, whose rounds take time in
// proportion to the workgroups they run).
uint64_t persistent_grid(const void* kernel, uint64_t blocks_needed, int block_size = 256, bool balance_rounds = false);

// Grid of the staged-stage encoder: persistent_grid, except for calls of at least PITCH_ENC_MIN_ROUNDS resident rounds,
// which run about 8 blocks per workgroup in one launch (many more workgroups than the CUs hold at once, handed
// out by the hardware as earlier ones finish). Measured on the config-5 value encode (524,288 blocks, 768
// resident workgroups): 4.84 TB/s persistent, 5.21 / 5.29 / 5.26 / 4.90 TB/s at 43 / 11 / 5.3 / 2.7 blocks per
// workgroup; on two more boxes, three repeats each, 8 blocks 1.5 % faster than 6, 10 or 12. Calls of fewer rounds
// lose from it (config 2, 8 rounds: -5 to -15 %; with the fair wave priority of persistent launches, calls of up
// to 48 rounds), so they stay persistent.
uint64_t encode_grid(const void* kernel, uint64_t blocks_needed, int block_size = 256);

// Dynamic LDS bytes that hold a launch of `kernel` to at most per_cu resident workgroups per CU: enough LDS per
// workgroup, with the kernel's own, that per_cu + 1 workgroups do not fit in a CU's LDS. 0 when per_cu is 0 or
// less, when the kernel's own LDS already holds it there, or when the bytes needed exceed a workgroup's maximum.
uint32_t lds_cap_bytes(const void* kernel, int per_cu);

// Rounds (grid-stride iterations per workgroup) per launch when a call of more rounds is split into several
// launches, or 0 for one launch: PITCH_SLICE_ROUNDS when it is 0 or more, else dflt.
uint64_t slice_rounds(uint64_t dflt);

// Smallest call (vectors) the float32 D = 1024 decode issues through the streaming decoder (PITCH_STREAM_MIN_VECTORS).
// Both decoders write the same bytes, so the threshold changes only the speed.
uint64_t stream_decode_min_vectors();

// Per-vector launch for one dimension D and I/O element type IO (0 float32, 1 float16, 2 bfloat16); one
// object file per (D, IO) defines launch_vec_d<D>_io<IO>, the batched encode launch_vec_batch_d<D>_io<IO> and the
// batched decode launch_vec_dec_batch_d<D>_io<IO>. The batched launches fill block_start themselves: the caller
// sets items and the segments.
#define PITCH_DECLARE_VEC_LAUNCH_IO(D, IO)                                                                     \
  hipError_t launch_vec_d##D##_io##IO(bool encode, bool polar, int bits, const VecArgs& a, hipStream_t s);      \
  hipError_t launch_vec_batch_d##D##_io##IO(bool polar, int bits, const VecBatchArgs& a, hipStream_t s);        \
  hipError_t launch_vec_dec_batch_d##D##_io##IO(bool polar, int bits, const DecBatchArgs& a, hipStream_t s);
#define PITCH_DECLARE_VEC_LAUNCH(D) \
  PITCH_DECLARE_VEC_LAUNCH_IO(D, 0) PITCH_DECLARE_VEC_LAUNCH_IO(D, 1) PITCH_DECLARE_VEC_LAUNCH_IO(D, 2)
PITCH_DECLARE_VEC_LAUNCH(2)
PITCH_DECLARE_VEC_LAUNCH(4)
PITCH_DECLARE_VEC_LAUNCH(8)
PITCH_DECLARE_VEC_LAUNCH(16)
PITCH_DECLARE_VEC_LAUNCH(32)
PITCH_DECLARE_VEC_LAUNCH(64)
PITCH_DECLARE_VEC_LAUNCH(128)
PITCH_DECLARE_VEC_LAUNCH(256)
PITCH_DECLARE_VEC_LAUNCH(512)
PITCH_DECLARE_VEC_LAUNCH(1024)
#undef PITCH_DECLARE_VEC_LAUNCH
#undef PITCH_DECLARE_VEC_LAUNCH_IO

// Per-channel launch for one I/O element type; one object file per IO defines launch_channel_io<IO>.
hipError_t launch_channel_io0(bool encode, int bits, const ChanArgs& a, hipStream_t s);
hipError_t launch_channel_io1(bool encode, int bits, const ChanArgs& a, hipStream_t s);
hipError_t launch_channel_io2(bool encode, int bits, const ChanArgs& a, hipStream_t s);
hipError_t launch_pack(bool pack, const PackArgs& a, hipStream_t s);
// Counts per thread (threads a multiple of 256) of the floats with bit patterns in [first, end) whose rcp_rn
// is not the correctly rounded reciprocal.
hipError_t launch_selftest_reciprocal(uint32_t* counts, uint32_t threads, uint32_t first, uint32_t end,
                                      hipStream_t s);

}  // namespace pitch
