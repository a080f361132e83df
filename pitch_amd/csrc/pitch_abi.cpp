// C ABI of libpitch_amd.so: argument validation and kernel dispatch (declared in include/pitch_amd.h).
//
// Validation mirrors the reference's launch contract before any GPU work is issued:
//   QuantConfig.init (Sources/PITCH/Models/QuantConfig.swift:24-35), ChannelQuantConfig.init
//   (Sources/PITCH/PerChannel.swift:30-43), Codec.params/check (Sources/PITCH/Core/Codec.swift:28-47) and
//   ChannelCodec.params/check (Sources/PITCH/PerChannel.swift:309-328).
// The reference's 32-bit limit on count * dim is lifted (64-bit counts and offsets).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <vector>
#include <string>
#include <unordered_map>

#include "../../include/pitch_amd.h"
#include "pitch_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return PITCH_OK;
}

bool is_pow2(uint32_t x) { return x != 0 && (x & (x - 1)) == 0; }

int validate_config(const pitch_config_t* c) {
  if (!c) return fail(PITCH_ERR_INVALID_INPUT, "config is null");
  if (c->method != PITCH_METHOD_TURBO && c->method != PITCH_METHOD_POLAR)
    return fail(PITCH_ERR_INVALID_INPUT, "unknown method %u", c->method);
  if (c->dim < 2 || c->dim > 1024 || !is_pow2(c->dim))
    return fail(PITCH_ERR_INVALID_DIMENSION, "Invalid dimension %u. Must be a power of two in [2, 1024].", c->dim);
  if (c->bits < 2 || c->bits > 8)
    return fail(PITCH_ERR_INVALID_BIT_WIDTH, "Invalid bit width %u. Must be in 2...8.", c->bits);
  return PITCH_OK;
}

int validate_channel_config(const pitch_channel_config_t* c) {
  if (!c) return fail(PITCH_ERR_INVALID_INPUT, "config is null");
  if (c->dim < 1 || c->dim > 1024)
    return fail(PITCH_ERR_INVALID_INPUT, "per-channel dimension %u must be in 1...1024", c->dim);
  if (c->bits < 2 || c->bits > 8)
    return fail(PITCH_ERR_INVALID_BIT_WIDTH, "Invalid bit width %u. Must be in 2...8.", c->bits);
  if (c->group_size < 1 || c->group_size > 65536)
    return fail(PITCH_ERR_INVALID_INPUT, "group size %u must be in 1...65536", c->group_size);
  return PITCH_OK;
}

uint32_t code_stride_of(uint32_t dim, uint32_t bits) { return (dim * bits + 31u) / 32u * 4u; }

// Offset alignment and "needs N bytes after offset" (Codec.swift:37-47). Offsets a caller passes must be multiples
// of 4 bytes, as in the reference; offsets the library derives itself may need only element alignment (align).
int check_buffer(const void* ptr, uint64_t bytes, uint64_t off, uint64_t need, const char* name, uint64_t align = 4) {
  if (!ptr) return fail(PITCH_ERR_INVALID_INPUT, "%s buffer is null", name);
  if (off % align != 0)
    return fail(PITCH_ERR_INVALID_INPUT, "%s offset %llu must be a non-negative multiple of %llu", name,
                (unsigned long long)off, (unsigned long long)align);
  if (bytes < off || bytes - off < need)
    return fail(PITCH_ERR_INVALID_INPUT, "%s buffer has %lld bytes after offset; needs %llu", name,
                (long long)bytes - (long long)off, (unsigned long long)need);
  return PITCH_OK;
}

// The buffer must be memory of the current device (Codec.swift:38-40 checks buffer.device).
int check_device(const void* ptr, int dev, const char* name) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return fail(PITCH_ERR_INVALID_INPUT, "%s buffer is not device memory", name);
  }
  if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged && !attr.isManaged)
    return fail(PITCH_ERR_INVALID_INPUT, "%s buffer is not device memory", name);
  if (attr.type == hipMemoryTypeDevice && attr.device != dev)
    return fail(PITCH_ERR_INVALID_INPUT, "%s buffer belongs to device %d, not the current device %d", name,
                attr.device, dev);
  return PITCH_OK;
}

// Scratch memory of pitch_enqueue_attention_decode_noalloc: the attention workspace for callers that cannot
// allocate device memory. One copy per device, held until the process ends; every call on a device shares it.
// Its device address comes from hipGetSymbolAddress (the array's name is only a host-side stand-in), looked up
// by the first call of any entry point that launches work on the device (current_device), so that a caller who
// captures a graph after any eager call on the device makes no lookup inside the capture.
constexpr uint64_t kNoAllocScratchBytes = PITCH_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on device dev, which must be the current device (looked up once per device).
int scratch_address(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return fail(PITCH_ERR_DEVICE_UNAVAILABLE, "device %d is out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail(PITCH_ERR_DEVICE_UNAVAILABLE, "scratch memory of device %d is unavailable: %s", dev,
                    hipGetErrorString(e));
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return PITCH_OK;
}

// The current device; the first call on a device also looks up its scratch array (scratch_address).
int current_device(int* dev) {
  if (hipGetDevice(dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(PITCH_ERR_DEVICE_UNAVAILABLE, "no HIP device is available");
  }
  void* unused = nullptr;
  return scratch_address(*dev, &unused);
}

bool mul_overflows(uint64_t a, uint64_t b) { return b != 0 && a > UINT64_MAX / b; }

#define PITCH_TRY(expr)       \
  do {                        \
    const int rc_ = (expr);   \
    if (rc_ != PITCH_OK) return rc_; \
  } while (0)

template <typename T>
T* at(const void* base, uint64_t off) {
  return (T*)((const char*)base + off);
}

using VecLaunch = hipError_t (*)(bool, bool, int, const pitch::VecArgs&, hipStream_t);

#define PITCH_VEC_ROW(D) {pitch::launch_vec_d##D##_io0, pitch::launch_vec_d##D##_io1, pitch::launch_vec_d##D##_io2}
constexpr VecLaunch kVecLaunch[10][3] = {PITCH_VEC_ROW(2),   PITCH_VEC_ROW(4),   PITCH_VEC_ROW(8),  PITCH_VEC_ROW(16),
                                         PITCH_VEC_ROW(32),  PITCH_VEC_ROW(64),  PITCH_VEC_ROW(128), PITCH_VEC_ROW(256),
                                         PITCH_VEC_ROW(512), PITCH_VEC_ROW(1024)};
#undef PITCH_VEC_ROW

hipError_t launch_vec(uint32_t dim, uint32_t io, bool encode, bool polar, int bits, const pitch::VecArgs& a,
                      hipStream_t s) {
  if (!is_pow2(dim) || dim < 2 || dim > 1024 || io > 2) return hipErrorInvalidValue;
  int li = 0;
  while ((2u << li) < dim) ++li;
  return kVecLaunch[li][io](encode, polar, bits, a, s);
}

using VecBatchLaunch = hipError_t (*)(bool, int, const pitch::VecBatchArgs&, hipStream_t);

#define PITCH_VEC_ROW(D) \
  {pitch::launch_vec_batch_d##D##_io0, pitch::launch_vec_batch_d##D##_io1, pitch::launch_vec_batch_d##D##_io2}
constexpr VecBatchLaunch kVecBatchLaunch[10][3] = {
    PITCH_VEC_ROW(2),  PITCH_VEC_ROW(4),   PITCH_VEC_ROW(8),   PITCH_VEC_ROW(16),  PITCH_VEC_ROW(32),
    PITCH_VEC_ROW(64), PITCH_VEC_ROW(128), PITCH_VEC_ROW(256), PITCH_VEC_ROW(512), PITCH_VEC_ROW(1024)};
#undef PITCH_VEC_ROW

using DecBatchLaunch = hipError_t (*)(bool, int, const pitch::DecBatchArgs&, hipStream_t);
#define PITCH_VEC_ROW(D) \
  {pitch::launch_vec_dec_batch_d##D##_io0, pitch::launch_vec_dec_batch_d##D##_io1, pitch::launch_vec_dec_batch_d##D##_io2}
constexpr DecBatchLaunch kDecBatchLaunch[10][3] = {
    PITCH_VEC_ROW(2),  PITCH_VEC_ROW(4),   PITCH_VEC_ROW(8),   PITCH_VEC_ROW(16),  PITCH_VEC_ROW(32),
    PITCH_VEC_ROW(64), PITCH_VEC_ROW(128), PITCH_VEC_ROW(256), PITCH_VEC_ROW(512), PITCH_VEC_ROW(1024)};
#undef PITCH_VEC_ROW

int dim_index(uint32_t dim) {
  int li = 0;
  while ((2u << li) < dim) ++li;
  return li;
}

hipError_t launch_channel(uint32_t io, bool encode, int bits, const pitch::ChanArgs& a, hipStream_t s) {
  switch (io) {
    case PITCH_IO_F32: return pitch::launch_channel_io0(encode, bits, a, s);
    case PITCH_IO_F16: return pitch::launch_channel_io1(encode, bits, a, s);
    case PITCH_IO_BF16: return pitch::launch_channel_io2(encode, bits, a, s);
    default: return hipErrorInvalidValue;
  }
}

// Bytes per element of an uncompressed buffer, or 0 for an unknown type.
uint32_t io_bytes(uint32_t io) { return io == PITCH_IO_F32 ? 4u : (io == PITCH_IO_F16 || io == PITCH_IO_BF16 ? 2u : 0u); }

int check_io(uint32_t io) {
  if (io_bytes(io) == 0) return fail(PITCH_ERR_INVALID_INPUT, "unknown element type %u", io);
  return PITCH_OK;
}

// Checks the sizes of a key-bias description for count vectors of dimension dim (no device access).
int check_key_bias(const pitch_key_bias_t* kb, uint32_t dim, uint64_t count) {
  if (!kb) return PITCH_OK;
  if (kb->heads < 1) return fail(PITCH_ERR_INVALID_INPUT, "key bias heads must be at least 1");
  PITCH_TRY(check_buffer(kb->bias, kb->bias_bytes, 0, (uint64_t)kb->heads * dim * 4u, "key bias"));
  const uint64_t tokens = (count + kb->heads - 1) / kb->heads;
  const uint64_t rows = kb->table_bytes / (4ull * dim);
  if (kb->first_position > rows || rows - kb->first_position < tokens)
    return fail(PITCH_ERR_INVALID_INPUT, "RoPE tables hold %llu positions; the call needs %llu from position %llu",
                (unsigned long long)rows, (unsigned long long)tokens, (unsigned long long)kb->first_position);
  PITCH_TRY(check_buffer(kb->cos, kb->table_bytes, 0, 0, "RoPE cos"));
  PITCH_TRY(check_buffer(kb->sin, kb->table_bytes, 0, 0, "RoPE sin"));
  return PITCH_OK;
}

// Checks that the key-bias tables are memory of the device and fills the launch fields.
int apply_key_bias(const pitch_key_bias_t* kb, int dev, pitch::VecArgs* a) {
  if (!kb) return PITCH_OK;
  PITCH_TRY(check_device(kb->bias, dev, "key bias"));
  PITCH_TRY(check_device(kb->cos, dev, "RoPE cos"));
  PITCH_TRY(check_device(kb->sin, dev, "RoPE sin"));
  a->kb_bias = (const float*)kb->bias;
  a->kb_cos = (const float*)kb->cos;
  a->kb_sin = (const float*)kb->sin;
  a->kb_first = kb->first_position;
  a->kb_heads = kb->heads;
  return PITCH_OK;
}

int encode_impl(const pitch_config_t* config, uint32_t io, const void* input, uint64_t input_bytes,
                uint64_t input_offset, void* codes, uint64_t codes_bytes, uint64_t codes_offset, void* scales,
                uint64_t scales_bytes, uint64_t scales_offset, uint64_t count, void* stream,
                const pitch_key_bias_t* kb = nullptr) {
  PITCH_TRY(validate_config(config));
  PITCH_TRY(check_io(io));
  const uint32_t dim = config->dim, cs = code_stride_of(dim, config->bits);
  if (count < 1) return fail(PITCH_ERR_INVALID_INPUT, "count must be at least 1");
  if (mul_overflows(count, (uint64_t)dim * 4u)) return fail(PITCH_ERR_INVALID_INPUT, "count is too large");
  PITCH_TRY(check_buffer(input, input_bytes, input_offset, count * dim * io_bytes(io), "input"));
  PITCH_TRY(check_buffer(codes, codes_bytes, codes_offset, count * cs, "codes"));
  PITCH_TRY(check_buffer(scales, scales_bytes, scales_offset, count * 4u, "scales"));
  PITCH_TRY(check_key_bias(kb, dim, count));
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(input, dev, "input"));
  PITCH_TRY(check_device(codes, dev, "codes"));
  PITCH_TRY(check_device(scales, dev, "scales"));
  pitch::VecArgs a{};
  a.in = at<const char>(input, input_offset);
  a.codes_out = at<uint32_t>(codes, codes_offset);
  a.scales_out = at<float>(scales, scales_offset);
  a.count = count;
  a.seed = config->seed;
  PITCH_TRY(apply_key_bias(kb, dev, &a));
  const hipError_t e = launch_vec(dim, io, true, config->method == PITCH_METHOD_POLAR, (int)config->bits, a,
                                  (hipStream_t)stream);
  if (e != hipSuccess) return fail(PITCH_ERR_ENCODING_FAILED, "Encoding failed: %s", hipGetErrorString(e));
  return ok();
}

int encode_batch_impl(const pitch_config_t* config, uint32_t io, const pitch_encode_item_t* items, uint32_t n,
                      void* stream) {
  PITCH_TRY(validate_config(config));
  PITCH_TRY(check_io(io));
  if (n < 1) return fail(PITCH_ERR_INVALID_INPUT, "a batch needs at least one segment");
  if (!items) return fail(PITCH_ERR_INVALID_INPUT, "segment array is null");
  const uint32_t dim = config->dim, cs = code_stride_of(dim, config->bits);
  for (uint32_t i = 0; i < n; ++i) {
    const pitch_encode_item_t& it = items[i];
    if (it.count < 1) return fail(PITCH_ERR_INVALID_INPUT, "segment %u: count must be at least 1", i);
    if (mul_overflows(it.count, (uint64_t)dim * 4u))
      return fail(PITCH_ERR_INVALID_INPUT, "segment %u: count is too large", i);
    PITCH_TRY(check_buffer(it.input, it.input_bytes, it.input_offset, it.count * dim * io_bytes(io), "input"));
    PITCH_TRY(check_buffer(it.codes, it.codes_bytes, it.codes_offset, it.count * cs, "codes"));
    PITCH_TRY(check_buffer(it.scales, it.scales_bytes, it.scales_offset, it.count * 4u, "scales"));
  }
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  for (uint32_t i = 0; i < n; ++i) {
    const pitch_encode_item_t& it = items[i];
    PITCH_TRY(check_device(it.input, dev, "input"));
    PITCH_TRY(check_device(it.codes, dev, "codes"));
    PITCH_TRY(check_device(it.scales, dev, "scales"));
  }
  const int li = dim_index(dim);
  pitch::VecBatchArgs a{};
  a.common.seed = config->seed;
  for (uint32_t i0 = 0; i0 < n; i0 += pitch::kBatchItems) {
    const uint32_t m = n - i0 < pitch::kBatchItems ? n - i0 : pitch::kBatchItems;
    a.items = m;  // the launcher assigns the segments their workgroups (block_start)
    for (uint32_t j = 0; j < m; ++j) {
      const pitch_encode_item_t& it = items[i0 + j];
      a.in[j] = at<const char>(it.input, it.input_offset);
      a.codes_out[j] = at<uint32_t>(it.codes, it.codes_offset);
      a.scales_out[j] = at<float>(it.scales, it.scales_offset);
      a.count[j] = it.count;
    }
    const hipError_t e = kVecBatchLaunch[li][io](config->method == PITCH_METHOD_POLAR, (int)config->bits, a,
                                                (hipStream_t)stream);
    if (e != hipSuccess) return fail(PITCH_ERR_ENCODING_FAILED, "Encoding failed: %s", hipGetErrorString(e));
  }
  return ok();
}

// Segments of a batched decode with at least this many vectors get a launch of their own (that of a single call).
constexpr uint64_t kDecBatchOwnLaunch = 1u << 18;

int decode_batch_impl(const pitch_config_t* config, uint32_t io, const pitch_decode_item_t* items, uint32_t n,
                      void* stream) {
  PITCH_TRY(validate_config(config));
  PITCH_TRY(check_io(io));
  if (n < 1) return fail(PITCH_ERR_INVALID_INPUT, "a batch needs at least one segment");
  if (!items) return fail(PITCH_ERR_INVALID_INPUT, "segment array is null");
  const uint32_t dim = config->dim, cs = code_stride_of(dim, config->bits);
  for (uint32_t i = 0; i < n; ++i) {
    const pitch_decode_item_t& it = items[i];
    if (it.count < 1) return fail(PITCH_ERR_INVALID_INPUT, "segment %u: count must be at least 1", i);
    if (mul_overflows(it.count, (uint64_t)dim * 4u))
      return fail(PITCH_ERR_INVALID_INPUT, "segment %u: count is too large", i);
    PITCH_TRY(check_buffer(it.codes, it.codes_bytes, it.codes_offset, it.count * cs, "codes"));
    PITCH_TRY(check_buffer(it.scales, it.scales_bytes, it.scales_offset, it.count * 4u, "scales"));
    PITCH_TRY(check_buffer(it.output, it.output_bytes, it.output_offset, it.count * dim * io_bytes(io), "output"));
  }
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  for (uint32_t i = 0; i < n; ++i) {
    const pitch_decode_item_t& it = items[i];
    PITCH_TRY(check_device(it.codes, dev, "codes"));
    PITCH_TRY(check_device(it.scales, dev, "scales"));
    PITCH_TRY(check_device(it.output, dev, "output"));
  }
  const int li = dim_index(dim);
  const bool polar = config->method == PITCH_METHOD_POLAR;
  pitch::DecBatchArgs a{};
  a.common.seed = config->seed;
  uint32_t m = 0;
  auto flush = [&]() -> hipError_t {
    if (m == 0) return hipSuccess;
    a.items = m;  // the launcher assigns the segments their workgroups (block_start)
    m = 0;
    return kDecBatchLaunch[li][io](polar, (int)config->bits, a, (hipStream_t)stream);
  };
  for (uint32_t i = 0; i < n; ++i) {
    const pitch_decode_item_t& it = items[i];
    hipError_t e = hipSuccess;
    if (it.count >= kDecBatchOwnLaunch) {
      // a long segment runs as the single call of it would: the batched kernel's larger argument block (1.4 KB
      // against 0.5 KB) measured 10 points slower over the half million workgroups of a 2^25-vector segment
      pitch::VecArgs v{};
      v.codes_in = at<const uint32_t>(it.codes, it.codes_offset);
      v.scales_in = at<const float>(it.scales, it.scales_offset);
      v.out = at<char>(it.output, it.output_offset);
      v.count = it.count;
      v.seed = config->seed;
      e = launch_vec(dim, io, false, polar, (int)config->bits, v, (hipStream_t)stream);
    } else {
      a.codes_in[m] = at<const uint32_t>(it.codes, it.codes_offset);
      a.scales_in[m] = at<const float>(it.scales, it.scales_offset);
      a.out[m] = at<char>(it.output, it.output_offset);
      a.count[m] = it.count;
      if (++m == pitch::kBatchItems) e = flush();
    }
    if (e != hipSuccess) return fail(PITCH_ERR_DECODING_FAILED, "Decoding failed: %s", hipGetErrorString(e));
  }
  const hipError_t e = flush();
  if (e != hipSuccess) return fail(PITCH_ERR_DECODING_FAILED, "Decoding failed: %s", hipGetErrorString(e));
  return ok();
}

int decode_impl(const pitch_config_t* config, uint32_t io, const void* codes, uint64_t codes_bytes,
                uint64_t codes_offset, const void* scales, uint64_t scales_bytes, uint64_t scales_offset,
                void* output, uint64_t output_bytes, uint64_t output_offset, uint64_t count, void* stream,
                const pitch_key_bias_t* kb = nullptr) {
  PITCH_TRY(validate_config(config));
  PITCH_TRY(check_io(io));
  const uint32_t dim = config->dim, cs = code_stride_of(dim, config->bits);
  if (count < 1) return fail(PITCH_ERR_INVALID_INPUT, "count must be at least 1");
  if (mul_overflows(count, (uint64_t)dim * 4u)) return fail(PITCH_ERR_INVALID_INPUT, "count is too large");
  PITCH_TRY(check_buffer(codes, codes_bytes, codes_offset, count * cs, "codes"));
  PITCH_TRY(check_buffer(scales, scales_bytes, scales_offset, count * 4u, "scales"));
  PITCH_TRY(check_buffer(output, output_bytes, output_offset, count * dim * io_bytes(io), "output"));
  PITCH_TRY(check_key_bias(kb, dim, count));
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(codes, dev, "codes"));
  PITCH_TRY(check_device(scales, dev, "scales"));
  PITCH_TRY(check_device(output, dev, "output"));
  pitch::VecArgs a{};
  a.codes_in = at<const uint32_t>(codes, codes_offset);
  a.scales_in = at<const float>(scales, scales_offset);
  a.out = at<char>(output, output_offset);
  a.count = count;
  a.seed = config->seed;
  PITCH_TRY(apply_key_bias(kb, dev, &a));
  const hipError_t e = launch_vec(dim, io, false, config->method == PITCH_METHOD_POLAR, (int)config->bits, a,
                                  (hipStream_t)stream);
  if (e != hipSuccess) return fail(PITCH_ERR_DECODING_FAILED, "Decoding failed: %s", hipGetErrorString(e));
  return ok();
}

// input_align: alignment the input offset needs (4 for a caller's offset; the element size for the offset
// pitch_enqueue_channel_append derives, which for 16-bit keys of a dimension that is not a multiple of 4 can be
// 2 mod 4 and is read element by element by the kernel such shapes use).
int channel_encode_impl(const pitch_channel_config_t* config, uint32_t io, const void* input, uint64_t input_bytes,
                        uint64_t input_offset, void* codes, uint64_t codes_bytes, uint64_t codes_offset,
                        void* ranges, uint64_t ranges_bytes, uint64_t ranges_offset, uint64_t count, void* stream,
                        uint64_t input_align = 4) {
  PITCH_TRY(validate_channel_config(config));
  PITCH_TRY(check_io(io));
  const uint32_t dim = config->dim, cs = code_stride_of(dim, config->bits);
  if (count < 1) return fail(PITCH_ERR_INVALID_INPUT, "count must be at least 1");
  if (count > 0xFFFFFFFFull) return fail(PITCH_ERR_INVALID_INPUT, "per-channel count must be below 2^32 tokens");
  const uint64_t groups = (count + config->group_size - 1) / config->group_size;
  PITCH_TRY(check_buffer(input, input_bytes, input_offset, count * dim * io_bytes(io), "input", input_align));
  PITCH_TRY(check_buffer(codes, codes_bytes, codes_offset, count * cs, "codes"));
  PITCH_TRY(check_buffer(ranges, ranges_bytes, ranges_offset, groups * 4u * dim, "ranges"));
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(input, dev, "input"));
  PITCH_TRY(check_device(codes, dev, "codes"));
  PITCH_TRY(check_device(ranges, dev, "ranges"));
  pitch::ChanArgs a{};
  a.in = at<const char>(input, input_offset);
  a.codes_out = at<uint32_t>(codes, codes_offset);
  a.ranges_out = at<uint16_t>(ranges, ranges_offset);
  a.count = (uint32_t)count;
  a.dim = dim;
  a.group = config->group_size;
  a.nwords = cs / 4u;
  const hipError_t e = launch_channel(io, true, (int)config->bits, a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(PITCH_ERR_ENCODING_FAILED, "Encoding failed: %s", hipGetErrorString(e));
  return ok();
}

int channel_decode_impl(const pitch_channel_config_t* config, uint32_t io, const void* codes, uint64_t codes_bytes,
                        uint64_t codes_offset, const void* ranges, uint64_t ranges_bytes, uint64_t ranges_offset,
                        void* output, uint64_t output_bytes, uint64_t output_offset, uint64_t count, void* stream) {
  PITCH_TRY(validate_channel_config(config));
  PITCH_TRY(check_io(io));
  const uint32_t dim = config->dim, cs = code_stride_of(dim, config->bits);
  if (count < 1) return fail(PITCH_ERR_INVALID_INPUT, "count must be at least 1");
  if (count > 0xFFFFFFFFull) return fail(PITCH_ERR_INVALID_INPUT, "per-channel count must be below 2^32 tokens");
  const uint64_t groups = (count + config->group_size - 1) / config->group_size;
  PITCH_TRY(check_buffer(codes, codes_bytes, codes_offset, count * cs, "codes"));
  PITCH_TRY(check_buffer(ranges, ranges_bytes, ranges_offset, groups * 4u * dim, "ranges"));
  PITCH_TRY(check_buffer(output, output_bytes, output_offset, count * dim * io_bytes(io), "output"));
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(codes, dev, "codes"));
  PITCH_TRY(check_device(ranges, dev, "ranges"));
  PITCH_TRY(check_device(output, dev, "output"));
  pitch::ChanArgs a{};
  a.codes_in = at<const uint32_t>(codes, codes_offset);
  a.ranges_in = at<const uint16_t>(ranges, ranges_offset);
  a.out = at<char>(output, output_offset);
  a.count = (uint32_t)count;
  a.dim = dim;
  a.group = config->group_size;
  a.nwords = cs / 4u;
  const hipError_t e = launch_channel(io, false, (int)config->bits, a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(PITCH_ERR_DECODING_FAILED, "Decoding failed: %s", hipGetErrorString(e));
  return ok();
}

uint32_t padded_queries(uint32_t nq) { return nq <= 1 ? 1u : (nq <= 2 ? 2u : (nq <= 4 ? 4u : 8u)); }

int validate_attention(const pitch_config_t* k, const pitch_config_t* v, const pitch_attention_desc_t* d) {
  PITCH_TRY(validate_config(k));
  PITCH_TRY(validate_config(v));
  if (!d) return fail(PITCH_ERR_INVALID_INPUT, "attention descriptor is null");
  if (k->dim != v->dim)
    return fail(PITCH_ERR_CONFIGURATION_MISMATCH, "key dimension %u and value dimension %u differ", k->dim, v->dim);
  if (k->dim != 64 && k->dim != 128)
    return fail(PITCH_ERR_INVALID_DIMENSION, "attention over compressed caches supports dimension 64 or 128, got %u",
                k->dim);
  if (d->q_per_kv < 1 || d->q_per_kv > 8)
    return fail(PITCH_ERR_INVALID_INPUT, "query heads per KV head %u must be in 1...8", d->q_per_kv);
  if (d->kv_heads < 1 || d->kv_heads > 65535)
    return fail(PITCH_ERR_INVALID_INPUT, "KV heads %u must be in 1...65535", d->kv_heads);
  if (d->tokens < 1) return fail(PITCH_ERR_INVALID_INPUT, "tokens must be at least 1");
  if (d->tokens > (1ull << 36)) return fail(PITCH_ERR_INVALID_INPUT, "tokens is too large");
  if (!(d->scale == d->scale) || d->scale == __builtin_inff() || d->scale == -__builtin_inff())
    return fail(PITCH_ERR_INVALID_INPUT, "softmax scale must be finite");
  return PITCH_OK;
}

// Largest vector index the call touches, with overflow checks: (tokens - 1) * token_stride +
// (kv_heads - 1) * head_stride.
int attention_extent(const pitch_attention_desc_t* d, uint64_t* vectors) {
  const uint64_t a = d->tokens - 1, b = (uint64_t)d->kv_heads - 1;
  if (mul_overflows(a, d->token_stride) || mul_overflows(b, d->head_stride))
    return fail(PITCH_ERR_INVALID_INPUT, "cache strides overflow");
  const uint64_t x = a * d->token_stride, y = b * d->head_stride;
  if (x > UINT64_MAX - y - 1) return fail(PITCH_ERR_INVALID_INPUT, "cache strides overflow");
  *vectors = x + y + 1;
  if (mul_overflows(*vectors, 4096u)) return fail(PITCH_ERR_INVALID_INPUT, "cache strides overflow");
  return PITCH_OK;
}

}  // namespace

namespace pitch {

int device_cu_count() {
  static std::mutex mu;
  static std::unordered_map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 1;
  cache[dev] = n;
  return n;
}

uint32_t attention_chunk_tokens(uint64_t tokens, uint32_t kv_heads) {
  // The largest chunk that still gives at least PITCH_ATTN_MIN_WG workgroups (512: two per compute unit; 1024 and
  // 2048 measured 0-51 % slower), between 128 and 1024 tokens; PITCH_ATTN_CHUNK (a compile-time tuning macro:
  // 64 ... 1024, a power of two) fixes it instead.
  static_assert(PITCH_ATTN_CHUNK == 0 ||
                    (PITCH_ATTN_CHUNK >= 64 && PITCH_ATTN_CHUNK <= 1024 && (PITCH_ATTN_CHUNK & (PITCH_ATTN_CHUNK - 1)) == 0),
                "PITCH_ATTN_CHUNK: 0 or a power of two in 64 ... 1024");
  if (PITCH_ATTN_CHUNK) return PITCH_ATTN_CHUNK;
  uint32_t chunk = 1024;
  while (chunk > 128 && (tokens + chunk - 1) / chunk * kv_heads < PITCH_ATTN_MIN_WG) chunk >>= 1;
  return chunk;
}

uint64_t attention_workspace_floats(uint32_t dim, uint32_t nqp, uint32_t kv_heads, uint64_t tokens, uint32_t chunk) {
  const uint64_t chunks = (tokens + chunk - 1) / chunk;
  return (uint64_t)kv_heads * nqp * (3 * dim + tokens + chunks * (2 + dim));
}

uint64_t slice_rounds(uint64_t dflt) { return PITCH_SLICE_ROUNDS >= 0 ? (uint64_t)PITCH_SLICE_ROUNDS : dflt; }

uint64_t stream_decode_min_vectors() { return (uint64_t)PITCH_STREAM_MIN_VECTORS; }

uint64_t persistent_grid(const void* kernel, uint64_t blocks_needed, int block_size, bool balance_rounds) {
  static std::mutex mu;
  static std::unordered_map<const void*, int> occ_cache;
  // PITCH_BLOCKS_PER_CU (a compile-time tuning macro) fixes the resident 256-thread-block count per CU
  // (smaller blocks scale it up); 0 = occupancy.
  int occ = 0;
  if (PITCH_BLOCKS_PER_CU > 0) {
    occ = PITCH_BLOCKS_PER_CU * (256 / block_size);
  } else {
    std::lock_guard<std::mutex> lock(mu);
    auto it = occ_cache.find(kernel);
    if (it != occ_cache.end()) {
      occ = it->second;
    } else {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, block_size, 0) != hipSuccess || occ < 1)
        occ = 1;
      occ_cache[kernel] = occ;
    }
  }
  const uint64_t cus = (uint64_t)device_cu_count();
  const uint64_t cap = cus * (uint64_t)occ;
  if (blocks_needed <= cap) return blocks_needed < 1 ? 1 : blocks_needed;
  if (!balance_rounds) return cap;
  // k workgroups per CU make ceil(need / (cus k)) rounds of k each; a bandwidth-bound round takes about k
  // times as long, so cost(k) = rounds * k counts the idle slots of a last, partly filled round. Take the
  // largest k in [occ / 2, occ] within 5 % of the cheapest: a call whose last round would be nearly empty
  // runs fewer, fully used rounds instead (e.g. 6144 blocks at 7 per CU on 256 CUs: 4 rounds of 6 rather than
  // 3.43 of 7; config-2 decode +4 %), while long calls keep full occupancy. Kernels bound by their arithmetic
  // lose more from fewer resident waves than they gain (16-bit per-channel encode -5 %), so callers opt in.
  const uint64_t kmin = ((uint64_t)occ + 1) / 2;
  auto cost = [&](uint64_t k) { return (blocks_needed + cus * k - 1) / (cus * k) * k; };
  uint64_t best = cost((uint64_t)occ);
  for (uint64_t k = kmin; k < (uint64_t)occ; ++k) best = cost(k) < best ? cost(k) : best;
  for (uint64_t k = (uint64_t)occ; k > kmin; --k)
    if (cost(k) * 20 <= best * 21) return cus * k;
  return cus * kmin;
}

uint32_t lds_cap_bytes(const void* kernel, int per_cu) {
  if (per_cu <= 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  // cached per (device, kernel, cap): the attributes do not change while the process runs
  struct Key {
    int dev;
    const void* kernel;
    int per_cu;
    bool operator==(const Key& o) const { return dev == o.dev && kernel == o.kernel && per_cu == o.per_cu; }
  };
  struct KeyHash {
    size_t operator()(const Key& k) const {
      return std::hash<const void*>()(k.kernel) ^ ((size_t)k.dev << 8) ^ ((size_t)k.per_cu << 16);
    }
  };
  static std::mutex mu;
  static std::unordered_map<Key, uint32_t, KeyHash> cache;
  const Key key{dev, kernel, per_cu};
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int cu_lds = 0, wg_lds = 0;
  hipFuncAttributes fa{};
  uint32_t bytes = 0;
  if (hipDeviceGetAttribute(&cu_lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) == hipSuccess &&
      hipDeviceGetAttribute(&wg_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && cu_lds > 0 &&
      hipFuncGetAttributes(&fa, kernel) == hipSuccess) {
    // more than 1 / (per_cu + 1) of the CU's LDS, in 512-byte allocation granules
    const uint64_t total = ((uint64_t)cu_lds / (uint64_t)(per_cu + 1) / 512u + 1u) * 512u;
    if ((uint64_t)fa.sharedSizeBytes < total && total <= (uint64_t)wg_lds) bytes = (uint32_t)(total - fa.sharedSizeBytes);
  }
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = bytes;
  return bytes;
}

uint64_t encode_grid(const void* kernel, uint64_t blocks_needed, int block_size) {
  // blocks per workgroup of long calls (PITCH_ENC_BLOCKS_PER_WG; 0 keeps every call persistent) and the resident
  // rounds from which a call is oversubscribed (PITCH_ENC_MIN_ROUNDS): compile-time tuning macros
  constexpr long per_wg = PITCH_ENC_BLOCKS_PER_WG, min_rounds = PITCH_ENC_MIN_ROUNDS;
  const uint64_t cap = persistent_grid(kernel, blocks_needed, block_size);
  if (per_wg <= 0 || blocks_needed < (uint64_t)(min_rounds > 1 ? min_rounds : 1) * cap) return cap;
  const uint64_t g = blocks_needed / (uint64_t)per_wg;
  return g > 0x7FFFFFFFull ? 0x7FFFFFFFull : (g < cap ? cap : g);
}

}  // namespace pitch

extern "C" {

uint32_t pitch_version(void) { return 0x000200u; }

const char* pitch_last_error(void) { return g_last_error.c_str(); }

int pitch_config(uint32_t method, uint32_t dim, uint32_t bits, uint32_t seed, pitch_config_t* out,
                 uint32_t* code_stride) {
  const pitch_config_t c{method, dim, bits, seed};
  PITCH_TRY(validate_config(&c));
  if (out) *out = c;
  if (code_stride) *code_stride = code_stride_of(dim, bits);
  return ok();
}

int pitch_channel_config(uint32_t dim, uint32_t bits, uint32_t group_size, pitch_channel_config_t* out,
                         uint32_t* code_stride, uint32_t* range_stride) {
  const pitch_channel_config_t c{dim, bits, group_size, 0u};
  PITCH_TRY(validate_channel_config(&c));
  if (out) *out = c;
  if (code_stride) *code_stride = code_stride_of(dim, bits);
  if (range_stride) *range_stride = 4u * dim;
  return ok();
}

int pitch_enqueue_encode(const pitch_config_t* config, const void* input, uint64_t input_bytes,
                         uint64_t input_offset, void* codes, uint64_t codes_bytes, uint64_t codes_offset,
                         void* scales, uint64_t scales_bytes, uint64_t scales_offset, uint64_t count,
                         void* stream) {
  return encode_impl(config, PITCH_IO_F32, input, input_bytes, input_offset, codes, codes_bytes, codes_offset,
                     scales, scales_bytes, scales_offset, count, stream);
}

int pitch_enqueue_encode_io(const pitch_config_t* config, uint32_t io_type, const void* input,
                            uint64_t input_bytes, uint64_t input_offset, void* codes, uint64_t codes_bytes,
                            uint64_t codes_offset, void* scales, uint64_t scales_bytes, uint64_t scales_offset,
                            uint64_t count, void* stream) {
  return encode_impl(config, io_type, input, input_bytes, input_offset, codes, codes_bytes, codes_offset, scales,
                     scales_bytes, scales_offset, count, stream);
}

int pitch_enqueue_encode_batch(const pitch_config_t* config, uint32_t io_type, const pitch_encode_item_t* items,
                               uint32_t n_items, void* stream) {
  return encode_batch_impl(config, io_type, items, n_items, stream);
}

int pitch_enqueue_decode_batch(const pitch_config_t* config, uint32_t io_type, const pitch_decode_item_t* items,
                               uint32_t n_items, void* stream) {
  return decode_batch_impl(config, io_type, items, n_items, stream);
}

int pitch_enqueue_decode(const pitch_config_t* config, const void* codes, uint64_t codes_bytes,
                         uint64_t codes_offset, const void* scales, uint64_t scales_bytes,
                         uint64_t scales_offset, void* output, uint64_t output_bytes, uint64_t output_offset,
                         uint64_t count, void* stream) {
  return decode_impl(config, PITCH_IO_F32, codes, codes_bytes, codes_offset, scales, scales_bytes, scales_offset,
                     output, output_bytes, output_offset, count, stream);
}

int pitch_enqueue_decode_io(const pitch_config_t* config, uint32_t io_type, const void* codes,
                            uint64_t codes_bytes, uint64_t codes_offset, const void* scales, uint64_t scales_bytes,
                            uint64_t scales_offset, void* output, uint64_t output_bytes, uint64_t output_offset,
                            uint64_t count, void* stream) {
  return decode_impl(config, io_type, codes, codes_bytes, codes_offset, scales, scales_bytes, scales_offset,
                     output, output_bytes, output_offset, count, stream);
}

int pitch_enqueue_encode_key_bias(const pitch_config_t* config, const pitch_key_bias_t* key_bias, const void* input,
                                  uint64_t input_bytes, uint64_t input_offset, void* codes, uint64_t codes_bytes,
                                  uint64_t codes_offset, void* scales, uint64_t scales_bytes, uint64_t scales_offset,
                                  uint64_t count, void* stream) {
  if (!key_bias) return fail(PITCH_ERR_INVALID_INPUT, "key bias is null");
  return encode_impl(config, PITCH_IO_F32, input, input_bytes, input_offset, codes, codes_bytes, codes_offset,
                     scales, scales_bytes, scales_offset, count, stream, key_bias);
}

int pitch_enqueue_decode_key_bias(const pitch_config_t* config, const pitch_key_bias_t* key_bias, const void* codes,
                                  uint64_t codes_bytes, uint64_t codes_offset, const void* scales,
                                  uint64_t scales_bytes, uint64_t scales_offset, void* output, uint64_t output_bytes,
                                  uint64_t output_offset, uint64_t count, void* stream) {
  if (!key_bias) return fail(PITCH_ERR_INVALID_INPUT, "key bias is null");
  return decode_impl(config, PITCH_IO_F32, codes, codes_bytes, codes_offset, scales, scales_bytes, scales_offset,
                     output, output_bytes, output_offset, count, stream, key_bias);
}

int pitch_enqueue_channel_encode(const pitch_channel_config_t* config, const void* input,
                                 uint64_t input_bytes, uint64_t input_offset, void* codes,
                                 uint64_t codes_bytes, uint64_t codes_offset, void* ranges,
                                 uint64_t ranges_bytes, uint64_t ranges_offset, uint64_t count,
                                 void* stream) {
  return channel_encode_impl(config, PITCH_IO_F32, input, input_bytes, input_offset, codes, codes_bytes,
                             codes_offset, ranges, ranges_bytes, ranges_offset, count, stream);
}

int pitch_enqueue_channel_encode_io(const pitch_channel_config_t* config, uint32_t io_type, const void* input,
                                    uint64_t input_bytes, uint64_t input_offset, void* codes,
                                    uint64_t codes_bytes, uint64_t codes_offset, void* ranges,
                                    uint64_t ranges_bytes, uint64_t ranges_offset, uint64_t count,
                                    void* stream) {
  return channel_encode_impl(config, io_type, input, input_bytes, input_offset, codes, codes_bytes, codes_offset,
                             ranges, ranges_bytes, ranges_offset, count, stream);
}

int pitch_enqueue_channel_decode(const pitch_channel_config_t* config, const void* codes,
                                 uint64_t codes_bytes, uint64_t codes_offset, const void* ranges,
                                 uint64_t ranges_bytes, uint64_t ranges_offset, void* output,
                                 uint64_t output_bytes, uint64_t output_offset, uint64_t count,
                                 void* stream) {
  return channel_decode_impl(config, PITCH_IO_F32, codes, codes_bytes, codes_offset, ranges, ranges_bytes,
                             ranges_offset, output, output_bytes, output_offset, count, stream);
}

int pitch_enqueue_channel_decode_io(const pitch_channel_config_t* config, uint32_t io_type, const void* codes,
                                    uint64_t codes_bytes, uint64_t codes_offset, const void* ranges,
                                    uint64_t ranges_bytes, uint64_t ranges_offset, void* output,
                                    uint64_t output_bytes, uint64_t output_offset, uint64_t count,
                                    void* stream) {
  return channel_decode_impl(config, io_type, codes, codes_bytes, codes_offset, ranges, ranges_bytes,
                             ranges_offset, output, output_bytes, output_offset, count, stream);
}

int pitch_enqueue_channel_append(const pitch_channel_config_t* config, uint32_t io_type, const void* input,
                                 uint64_t input_bytes, uint64_t input_offset, void* codes, uint64_t codes_bytes,
                                 uint64_t codes_offset, void* ranges, uint64_t ranges_bytes, uint64_t ranges_offset,
                                 uint64_t total_tokens, uint64_t new_tokens, void* stream) {
  PITCH_TRY(validate_channel_config(config));
  PITCH_TRY(check_io(io_type));
  if (new_tokens < 1) return fail(PITCH_ERR_INVALID_INPUT, "new tokens must be at least 1");
  if (total_tokens < new_tokens)
    return fail(PITCH_ERR_INVALID_INPUT, "total tokens %llu is below the %llu new tokens",
                (unsigned long long)total_tokens, (unsigned long long)new_tokens);
  if (total_tokens > 0xFFFFFFFFull) return fail(PITCH_ERR_INVALID_INPUT, "per-channel count must be below 2^32 tokens");
  const uint32_t dim = config->dim, G = config->group_size, cs = code_stride_of(dim, config->bits);
  const uint64_t esize = io_bytes(io_type);
  // the whole cache must fit its buffers, as for one encode of total_tokens tokens
  const uint64_t groups = (total_tokens + G - 1) / G;
  PITCH_TRY(check_buffer(input, input_bytes, input_offset, total_tokens * dim * esize, "input"));
  PITCH_TRY(check_buffer(codes, codes_bytes, codes_offset, total_tokens * cs, "codes"));
  PITCH_TRY(check_buffer(ranges, ranges_bytes, ranges_offset, groups * 4u * dim, "ranges"));
  // re-encode from the start of the group that holds the first new token
  const uint64_t g0 = (total_tokens - new_tokens) / G, first = g0 * G;
  // input_offset itself is a multiple of 4 (checked above); the derived offset is element-aligned
  return channel_encode_impl(config, io_type, input, input_bytes, input_offset + first * dim * esize, codes,
                             codes_bytes, codes_offset + first * cs, ranges, ranges_bytes,
                             ranges_offset + g0 * 4u * dim, total_tokens - first, stream, esize);
}

int pitch_attention_workspace_size(const pitch_config_t* key_config, const pitch_config_t* value_config,
                                   const pitch_attention_desc_t* desc, uint64_t* bytes) {
  PITCH_TRY(validate_attention(key_config, value_config, desc));
  if (!bytes) return fail(PITCH_ERR_INVALID_INPUT, "bytes is null");
  const uint32_t chunk = pitch::attention_chunk_tokens(desc->tokens, desc->kv_heads);
  *bytes = 4u * pitch::attention_workspace_floats(key_config->dim, padded_queries(desc->q_per_kv), desc->kv_heads,
                                                  desc->tokens, chunk);
  return ok();
}

}  // extern "C"

namespace {

// pitch_enqueue_attention_decode with either a caller's workspace or (workspace == nullptr) the library's scratch.
int attention_impl(const pitch_config_t* key_config, const pitch_config_t* value_config,
                   const pitch_attention_desc_t* desc, const void* q, uint64_t q_bytes, uint64_t q_offset,
                   const void* key_codes, uint64_t key_codes_bytes, uint64_t key_codes_offset, const void* key_scales,
                   uint64_t key_scales_bytes, uint64_t key_scales_offset, const void* value_codes,
                   uint64_t value_codes_bytes, uint64_t value_codes_offset, const void* value_scales,
                   uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output, uint64_t output_bytes,
                   uint64_t output_offset, void* lse, uint64_t lse_bytes, uint64_t lse_offset, void* workspace,
                   uint64_t workspace_bytes, void* stream, bool use_scratch,
                   const pitch_key_bias_t* kb = nullptr) {
  PITCH_TRY(validate_attention(key_config, value_config, desc));
  const uint32_t dim = key_config->dim, nq = desc->q_per_kv, nqp = padded_queries(nq);
  const uint32_t kcs = code_stride_of(dim, key_config->bits), vcs = code_stride_of(dim, value_config->bits);
  uint64_t vectors = 0;
  PITCH_TRY(attention_extent(desc, &vectors));
  const uint64_t queries = (uint64_t)desc->kv_heads * nq;
  PITCH_TRY(check_buffer(q, q_bytes, q_offset, queries * dim * 4u, "query"));
  PITCH_TRY(check_buffer(key_codes, key_codes_bytes, key_codes_offset, vectors * kcs, "key codes"));
  PITCH_TRY(check_buffer(key_scales, key_scales_bytes, key_scales_offset, vectors * 4u, "key scales"));
  PITCH_TRY(check_buffer(value_codes, value_codes_bytes, value_codes_offset, vectors * vcs, "value codes"));
  PITCH_TRY(check_buffer(value_scales, value_scales_bytes, value_scales_offset, vectors * 4u, "value scales"));
  PITCH_TRY(check_buffer(output, output_bytes, output_offset, queries * dim * 4u, "output"));
  if (lse) PITCH_TRY(check_buffer(lse, lse_bytes, lse_offset, queries * 4u, "lse"));
  if (kb) {
    if (kb->heads != desc->kv_heads)
      return fail(PITCH_ERR_INVALID_INPUT, "key bias has %u heads; the call has %u KV heads", kb->heads,
                  desc->kv_heads);
    PITCH_TRY(check_key_bias(kb, dim, desc->tokens * desc->kv_heads));  // positions first .. first + tokens - 1
  }
  const uint32_t chunk = pitch::attention_chunk_tokens(desc->tokens, desc->kv_heads);
  const uint64_t ws_need = 4u * pitch::attention_workspace_floats(dim, nqp, desc->kv_heads, desc->tokens, chunk);
  if (use_scratch) {
    if (ws_need > kNoAllocScratchBytes)
      return fail(PITCH_ERR_INVALID_INPUT,
                  "this call needs %llu bytes of workspace; the allocation-free entry point holds at most %llu "
                  "(pass a workspace to pitch_enqueue_attention_decode instead)",
                  (unsigned long long)ws_need, (unsigned long long)kNoAllocScratchBytes);
  } else {
    PITCH_TRY(check_buffer(workspace, workspace_bytes, 0, ws_need, "workspace"));
  }
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(q, dev, "query"));
  PITCH_TRY(check_device(key_codes, dev, "key codes"));
  PITCH_TRY(check_device(key_scales, dev, "key scales"));
  PITCH_TRY(check_device(value_codes, dev, "value codes"));
  PITCH_TRY(check_device(value_scales, dev, "value scales"));
  PITCH_TRY(check_device(output, dev, "output"));
  if (lse) PITCH_TRY(check_device(lse, dev, "lse"));
  if (use_scratch) PITCH_TRY(scratch_address(dev, &workspace));
  else PITCH_TRY(check_device(workspace, dev, "workspace"));
  if (kb) {
    PITCH_TRY(check_device(kb->bias, dev, "key bias"));
    PITCH_TRY(check_device(kb->cos, dev, "RoPE cos"));
    PITCH_TRY(check_device(kb->sin, dev, "RoPE sin"));
  }
  pitch::AttnArgs a{};
  a.q = at<const float>(q, q_offset);
  a.k_codes = at<const uint32_t>(key_codes, key_codes_offset);
  a.k_scales = at<const float>(key_scales, key_scales_offset);
  a.v_codes = at<const uint32_t>(value_codes, value_codes_offset);
  a.v_scales = at<const float>(value_scales, value_scales_offset);
  a.out = at<float>(output, output_offset);
  a.lse = lse ? at<float>(lse, lse_offset) : nullptr;
  a.ws = (float*)workspace;
  a.tokens = desc->tokens;
  a.token_stride = desc->token_stride;
  a.head_stride = desc->head_stride;
  a.dim = dim;
  a.nq = nq;
  a.nqp = nqp;
  a.kv_heads = desc->kv_heads;
  a.kbits = key_config->bits;
  a.vbits = value_config->bits;
  a.kpolar = key_config->method == PITCH_METHOD_POLAR;
  a.vpolar = value_config->method == PITCH_METHOD_POLAR;
  a.kseed = key_config->seed;
  a.vseed = value_config->seed;
  a.chunk = chunk;
  a.chunks = (uint32_t)((desc->tokens + chunk - 1) / chunk);
  // softmax scale, log2(e) (scores in log2 units) and the key decode's 1 / sqrt(d), folded into the query
  a.qscale = (float)((double)desc->scale * 1.4426950408889634 / __builtin_sqrt((double)dim));
  a.oscale = (float)(1.0 / __builtin_sqrt((double)dim));
  if (kb) {
    a.kb_bias = (const float*)kb->bias;
    a.kb_cos = (const float*)kb->cos;
    a.kb_sin = (const float*)kb->sin;
    a.kb_first = kb->first_position;
    a.kscale = (float)((double)desc->scale * 1.4426950408889634);  // the bias term is in the keys' own scale
  }
  const hipError_t e = dim == 64 ? pitch::launch_attention_d64(a, (hipStream_t)stream)
                                 : pitch::launch_attention_d128(a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(PITCH_ERR_DECODING_FAILED, "Attention failed: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int pitch_enqueue_attention_decode(const pitch_config_t* key_config, const pitch_config_t* value_config,
                                   const pitch_attention_desc_t* desc, const void* q, uint64_t q_bytes,
                                   uint64_t q_offset, const void* key_codes, uint64_t key_codes_bytes,
                                   uint64_t key_codes_offset, const void* key_scales, uint64_t key_scales_bytes,
                                   uint64_t key_scales_offset, const void* value_codes, uint64_t value_codes_bytes,
                                   uint64_t value_codes_offset, const void* value_scales,
                                   uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output,
                                   uint64_t output_bytes, uint64_t output_offset, void* lse, uint64_t lse_bytes,
                                   uint64_t lse_offset, void* workspace, uint64_t workspace_bytes, void* stream) {
  return attention_impl(key_config, value_config, desc, q, q_bytes, q_offset, key_codes, key_codes_bytes,
                        key_codes_offset, key_scales, key_scales_bytes, key_scales_offset, value_codes,
                        value_codes_bytes, value_codes_offset, value_scales, value_scales_bytes, value_scales_offset,
                        output, output_bytes, output_offset, lse, lse_bytes, lse_offset, workspace, workspace_bytes,
                        stream, false);
}

int pitch_enqueue_attention_decode_key_bias(
    const pitch_config_t* key_config, const pitch_config_t* value_config, const pitch_attention_desc_t* desc,
    const pitch_key_bias_t* key_bias, const void* q, uint64_t q_bytes, uint64_t q_offset, const void* key_codes,
    uint64_t key_codes_bytes, uint64_t key_codes_offset, const void* key_scales, uint64_t key_scales_bytes,
    uint64_t key_scales_offset, const void* value_codes, uint64_t value_codes_bytes, uint64_t value_codes_offset,
    const void* value_scales, uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output,
    uint64_t output_bytes, uint64_t output_offset, void* lse, uint64_t lse_bytes, uint64_t lse_offset,
    void* workspace, uint64_t workspace_bytes, void* stream) {
  if (!key_bias) return fail(PITCH_ERR_INVALID_INPUT, "key bias is null");
  return attention_impl(key_config, value_config, desc, q, q_bytes, q_offset, key_codes, key_codes_bytes,
                        key_codes_offset, key_scales, key_scales_bytes, key_scales_offset, value_codes,
                        value_codes_bytes, value_codes_offset, value_scales, value_scales_bytes, value_scales_offset,
                        output, output_bytes, output_offset, lse, lse_bytes, lse_offset, workspace, workspace_bytes,
                        stream, false, key_bias);
}

int pitch_enqueue_attention_decode_noalloc(const pitch_config_t* key_config, const pitch_config_t* value_config,
                                           const pitch_attention_desc_t* desc, const void* q, uint64_t q_bytes,
                                           uint64_t q_offset, const void* key_codes, uint64_t key_codes_bytes,
                                           uint64_t key_codes_offset, const void* key_scales,
                                           uint64_t key_scales_bytes, uint64_t key_scales_offset,
                                           const void* value_codes, uint64_t value_codes_bytes,
                                           uint64_t value_codes_offset, const void* value_scales,
                                           uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output,
                                           uint64_t output_bytes, uint64_t output_offset, void* lse,
                                           uint64_t lse_bytes, uint64_t lse_offset, void* stream) {
  return attention_impl(key_config, value_config, desc, q, q_bytes, q_offset, key_codes, key_codes_bytes,
                        key_codes_offset, key_scales, key_scales_bytes, key_scales_offset, value_codes,
                        value_codes_bytes, value_codes_offset, value_scales, value_scales_bytes, value_scales_offset,
                        output, output_bytes, output_offset, lse, lse_bytes, lse_offset, nullptr, 0, stream, true);
}

int pitch_attention_channel_keys_workspace_size(const pitch_channel_config_t* key_config,
                                                const pitch_config_t* value_config, const pitch_attention_desc_t* desc,
                                                uint64_t* bytes) {
  PITCH_TRY(validate_channel_config(key_config));
  if (!value_config) return fail(PITCH_ERR_INVALID_INPUT, "value config is null");
  const pitch_config_t k{PITCH_METHOD_TURBO, key_config->dim, key_config->bits, 0u};
  return pitch_attention_workspace_size(&k, value_config, desc, bytes);
}

int pitch_enqueue_attention_decode_channel_keys(
    const pitch_channel_config_t* key_config, const pitch_config_t* value_config, const pitch_attention_desc_t* desc,
    const void* q, uint64_t q_bytes, uint64_t q_offset, const void* key_codes, uint64_t key_codes_bytes,
    uint64_t key_codes_offset, const void* key_ranges, uint64_t key_ranges_bytes, uint64_t key_ranges_offset,
    const void* value_codes, uint64_t value_codes_bytes, uint64_t value_codes_offset, const void* value_scales,
    uint64_t value_scales_bytes, uint64_t value_scales_offset, void* output, uint64_t output_bytes,
    uint64_t output_offset, void* lse, uint64_t lse_bytes, uint64_t lse_offset, void* workspace,
    uint64_t workspace_bytes, void* stream) {
  PITCH_TRY(validate_channel_config(key_config));
  const pitch_config_t kvec{PITCH_METHOD_TURBO, key_config->dim, key_config->bits, 0u};
  PITCH_TRY(validate_attention(&kvec, value_config, desc));
  const uint32_t dim = key_config->dim, G = key_config->group_size, nq = desc->q_per_kv, nqp = padded_queries(nq);
  if (G % 64 != 0)
    return fail(PITCH_ERR_INVALID_INPUT, "attention over per-channel keys needs a group size that is a multiple of 64, "
                "got %u", G);
  if (desc->token_stride != 1)
    return fail(PITCH_ERR_INVALID_INPUT, "per-channel key caches are head-major: token_stride must be 1");
  if (desc->kv_heads > 1 && (desc->head_stride < desc->tokens || desc->head_stride % G != 0))
    return fail(PITCH_ERR_INVALID_INPUT, "head_stride %llu must hold the tokens and be a multiple of the group size %u",
                (unsigned long long)desc->head_stride, G);
  const uint64_t head_stride = desc->kv_heads > 1 ? desc->head_stride : (desc->tokens + G - 1) / G * G;
  const uint32_t kcs = code_stride_of(dim, key_config->bits), vcs = code_stride_of(dim, value_config->bits);
  uint64_t vectors = 0;
  PITCH_TRY(attention_extent(desc, &vectors));
  const uint64_t queries = (uint64_t)desc->kv_heads * nq;
  const uint64_t kgroups = ((uint64_t)(desc->kv_heads - 1) * head_stride + desc->tokens + G - 1) / G;
  PITCH_TRY(check_buffer(q, q_bytes, q_offset, queries * dim * 4u, "query"));
  PITCH_TRY(check_buffer(key_codes, key_codes_bytes, key_codes_offset, vectors * kcs, "key codes"));
  PITCH_TRY(check_buffer(key_ranges, key_ranges_bytes, key_ranges_offset, kgroups * 4u * dim, "key ranges"));
  PITCH_TRY(check_buffer(value_codes, value_codes_bytes, value_codes_offset, vectors * vcs, "value codes"));
  PITCH_TRY(check_buffer(value_scales, value_scales_bytes, value_scales_offset, vectors * 4u, "value scales"));
  PITCH_TRY(check_buffer(output, output_bytes, output_offset, queries * dim * 4u, "output"));
  if (lse) PITCH_TRY(check_buffer(lse, lse_bytes, lse_offset, queries * 4u, "lse"));
  const uint32_t chunk = pitch::attention_chunk_tokens(desc->tokens, desc->kv_heads);
  const uint64_t ws_need = 4u * pitch::attention_workspace_floats(dim, nqp, desc->kv_heads, desc->tokens, chunk);
  PITCH_TRY(check_buffer(workspace, workspace_bytes, 0, ws_need, "workspace"));
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(q, dev, "query"));
  PITCH_TRY(check_device(key_codes, dev, "key codes"));
  PITCH_TRY(check_device(key_ranges, dev, "key ranges"));
  PITCH_TRY(check_device(value_codes, dev, "value codes"));
  PITCH_TRY(check_device(value_scales, dev, "value scales"));
  PITCH_TRY(check_device(output, dev, "output"));
  if (lse) PITCH_TRY(check_device(lse, dev, "lse"));
  PITCH_TRY(check_device(workspace, dev, "workspace"));
  pitch::AttnArgs a{};
  a.q = at<const float>(q, q_offset);
  a.k_codes = at<const uint32_t>(key_codes, key_codes_offset);
  a.k_ranges = at<const uint16_t>(key_ranges, key_ranges_offset);
  a.k_group = G;
  a.v_codes = at<const uint32_t>(value_codes, value_codes_offset);
  a.v_scales = at<const float>(value_scales, value_scales_offset);
  a.out = at<float>(output, output_offset);
  a.lse = lse ? at<float>(lse, lse_offset) : nullptr;
  a.ws = (float*)workspace;
  a.tokens = desc->tokens;
  a.token_stride = 1;
  a.head_stride = head_stride;
  a.dim = dim;
  a.nq = nq;
  a.nqp = nqp;
  a.kv_heads = desc->kv_heads;
  a.kbits = key_config->bits;
  a.vbits = value_config->bits;
  a.vpolar = value_config->method == PITCH_METHOD_POLAR;
  a.vseed = value_config->seed;
  a.chunk = chunk;
  a.chunks = (uint32_t)((desc->tokens + chunk - 1) / chunk);
  a.kscale = (float)((double)desc->scale * 1.4426950408889634);
  a.oscale = (float)(1.0 / __builtin_sqrt((double)dim));
  const hipError_t e = dim == 64 ? pitch::launch_attention_d64(a, (hipStream_t)stream)
                                 : pitch::launch_attention_d128(a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(PITCH_ERR_DECODING_FAILED, "Attention failed: %s", hipGetErrorString(e));
  return ok();
}

static int pack_common(bool pack, uint32_t dim, uint32_t bits, const void* src, uint64_t src_bytes,
                       uint64_t src_off, void* dst, uint64_t dst_bytes, uint64_t dst_off, uint64_t count,
                       void* stream) {
  if (dim < 1 || dim > 1024) return fail(PITCH_ERR_INVALID_DIMENSION, "dimension %u must be in 1...1024", dim);
  if (bits < 2 || bits > 8) return fail(PITCH_ERR_INVALID_BIT_WIDTH, "Invalid bit width %u. Must be in 2...8.", bits);
  if (count < 1) return fail(PITCH_ERR_INVALID_INPUT, "count must be at least 1");
  if (mul_overflows(count, 4096u)) return fail(PITCH_ERR_INVALID_INPUT, "count is too large");
  const uint64_t packed = count * code_stride_of(dim, bits), unpacked = count * dim;
  if (pack) {
    PITCH_TRY(check_buffer(src, src_bytes, 0, 0, "unpacked"));
    if (src_bytes < src_off || src_bytes - src_off < unpacked)
      return fail(PITCH_ERR_INVALID_INPUT, "unpacked buffer needs %llu bytes after offset", (unsigned long long)unpacked);
    PITCH_TRY(check_buffer(dst, dst_bytes, dst_off, packed, "packed"));
  } else {
    PITCH_TRY(check_buffer(src, src_bytes, src_off, packed, "packed"));
    if (!dst) return fail(PITCH_ERR_INVALID_INPUT, "unpacked buffer is null");
    if (dst_bytes < dst_off || dst_bytes - dst_off < unpacked)
      return fail(PITCH_ERR_INVALID_INPUT, "unpacked buffer needs %llu bytes after offset", (unsigned long long)unpacked);
  }
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  PITCH_TRY(check_device(src, dev, pack ? "unpacked" : "packed"));
  PITCH_TRY(check_device(dst, dev, pack ? "packed" : "unpacked"));
  pitch::PackArgs a{};
  a.count = count;
  a.dim = dim;
  a.bits = bits;
  if (pack) {
    a.unpacked_in = at<const uint8_t>(src, src_off);
    a.packed_out = at<uint32_t>(dst, dst_off);
  } else {
    a.packed_in = at<const uint32_t>(src, src_off);
    a.unpacked_out = at<uint8_t>(dst, dst_off);
  }
  const hipError_t e = pitch::launch_pack(pack, a, (hipStream_t)stream);
  if (e != hipSuccess)
    return fail(pack ? PITCH_ERR_ENCODING_FAILED : PITCH_ERR_DECODING_FAILED, "%s failed: %s",
                pack ? "pack" : "unpack", hipGetErrorString(e));
  return ok();
}

int pitch_enqueue_pack_codes(uint32_t dim, uint32_t bits, const void* unpacked, uint64_t unpacked_bytes,
                             uint64_t unpacked_offset, void* packed, uint64_t packed_bytes,
                             uint64_t packed_offset, uint64_t count, void* stream) {
  return pack_common(true, dim, bits, unpacked, unpacked_bytes, unpacked_offset, packed, packed_bytes,
                     packed_offset, count, stream);
}

int pitch_enqueue_unpack_codes(uint32_t dim, uint32_t bits, const void* packed, uint64_t packed_bytes,
                               uint64_t packed_offset, void* unpacked, uint64_t unpacked_bytes,
                               uint64_t unpacked_offset, uint64_t count, void* stream) {
  return pack_common(false, dim, bits, packed, packed_bytes, packed_offset, unpacked, unpacked_bytes,
                     unpacked_offset, count, stream);
}

int pitch_selftest_reciprocal(uint64_t* mismatches) {
  if (!mismatches) return fail(PITCH_ERR_INVALID_INPUT, "mismatches is null");
  int dev = 0;
  PITCH_TRY(current_device(&dev));
  constexpr uint32_t kThreads = 1u << 20;
  constexpr uint32_t kFirst = 0x00800000u, kEnd = 0x7e800000u;  // positive normals below 2^126
  uint32_t* d = nullptr;
  if (hipMalloc((void**)&d, kThreads * sizeof(uint32_t)) != hipSuccess)
    return fail(PITCH_ERR_DEVICE_UNAVAILABLE, "self-test allocation failed");
  std::vector<uint32_t> h(kThreads);
  hipError_t e = pitch::launch_selftest_reciprocal(d, kThreads, kFirst, kEnd, nullptr);
  if (e == hipSuccess) e = hipMemcpy(h.data(), d, kThreads * sizeof(uint32_t), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(PITCH_ERR_ENCODING_FAILED, "self-test failed: %s", hipGetErrorString(e));
  uint64_t total = 0;
  for (uint32_t c : h) total += c;
  *mismatches = total;
  return ok();
}

}  // extern "C"
