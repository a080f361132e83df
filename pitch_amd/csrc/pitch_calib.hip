// Measurement kernels for bench.py (libpitch_calib.so): not part of the codec, and not declared in
// include/pitch_amd.h.
//
// calib_stream moves the bytes an encoder moves, with no arithmetic between its loads and its stores: each
// unit (one vector, or one token row of a key cache) is unit_bytes read and out_words 4-byte words written.
// The loads follow a chosen access shape, so the measured rate is the ceiling of that shape at that footprint:
// - seg_bytes: the contiguous piece of one unit that one load instruction reads per unit. A wave's load
//   instruction covers 64 * 16 / seg_bytes units, seg_bytes each; a unit takes unit_bytes / seg_bytes
//   instructions. The staged encoders read 64-byte pieces at d = 64 and 128-byte pieces at d = 128 (four or
//   eight lanes of 16 bytes per vector per instruction); the KIVI encoder reads 128-byte row pieces.
// - workgroups: the grid. Non-zero: a persistent grid of that many 256-thread workgroups striding over the
//   units (the encoders run 3 workgroups per CU); zero: one block of units per workgroup, all in one launch.
// - nontemporal: non-temporal loads and stores (the encoders use them), or cached ones.
// The stores are coalesced: a wave's units write one contiguous run of words, as the encoders' codes do.
// Every lane's loaded words feed a value that is compared before the stores, so the compiler keeps every load.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace pitch_calib {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr uint32_t kNever = 0x9E3779B9u;  // a fold value that stores to word 0 (keeps the loads live)

// L lanes read one unit's seg piece (L * 16 bytes); CPL pieces per unit (unit = L * CPL * 16 bytes).
template <int L, int CPL, bool NT>
__global__ __launch_bounds__(kBlock) void calib_stream(const u32x4* __restrict__ in, uint32_t* __restrict__ out,
                                                       uint64_t units, uint32_t out_words, uint64_t grid_blocks) {
  constexpr int UPW = 64 / L;  // units per wave and instruction
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ul = lane / L, pl = lane % L;
  const uint64_t wblocks = (units + UPW - 1) / UPW;
  for (uint64_t wb = (uint64_t)blockIdx.x * (kBlock / 64) + wave; wb < wblocks; wb += grid_blocks * (kBlock / 64)) {
    uint64_t u = wb * UPW + ul;
    if (u >= units) u = units - 1;  // the last wave block re-reads the last unit
    const u32x4* src = in + u * (uint64_t)(L * CPL) + pl;
    u32x4 c[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) c[i] = NT ? __builtin_nontemporal_load(src + i * L) : src[i * L];
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) acc ^= c[i].x ^ c[i].y ^ c[i].z ^ c[i].w;
    if (acc == kNever) out[0] = acc;
    // the wave's UPW units own one contiguous run of UPW * out_words words (as an encoder's codes): lane l
    // writes words l, l + 64, ... of it, up to the last unit's end
    const uint64_t w0 = wb * UPW * (uint64_t)out_words;
    const uint64_t wend = units * (uint64_t)out_words;
    const uint64_t run = (uint64_t)UPW * out_words;
    for (uint64_t j = lane; j < run && w0 + j < wend; j += 64) {
      if constexpr (NT) __builtin_nontemporal_store(acc + (uint32_t)j, out + w0 + j);
      else out[w0 + j] = acc + (uint32_t)j;
    }
  }
}

template <int L, int CPL>
hipError_t launch(const void* in, void* out, uint64_t units, uint32_t out_words, uint32_t workgroups, bool nt,
                  hipStream_t s) {
  constexpr int UPW = 64 / L;
  const uint64_t wblocks = (units + UPW - 1) / UPW;
  const uint64_t grid = workgroups ? (uint64_t)workgroups : (wblocks + kBlock / 64 - 1) / (kBlock / 64);
  if (grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
  if (nt)
    hipLaunchKernelGGL((calib_stream<L, CPL, true>), dim3((uint32_t)grid), dim3(kBlock), 0, s, (const u32x4*)in,
                       (uint32_t*)out, units, out_words, grid);
  else
    hipLaunchKernelGGL((calib_stream<L, CPL, false>), dim3((uint32_t)grid), dim3(kBlock), 0, s, (const u32x4*)in,
                       (uint32_t*)out, units, out_words, grid);
  return hipGetLastError();
}

template <int L>
hipError_t launch_cpl(uint32_t cpl, const void* in, void* out, uint64_t units, uint32_t out_words,
                      uint32_t workgroups, bool nt, hipStream_t s) {
  switch (cpl) {
    case 1: return launch<L, 1>(in, out, units, out_words, workgroups, nt, s);
    case 2: return launch<L, 2>(in, out, units, out_words, workgroups, nt, s);
    case 4: return launch<L, 4>(in, out, units, out_words, workgroups, nt, s);
    case 8: return launch<L, 8>(in, out, units, out_words, workgroups, nt, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pitch_calib

// Reads units * unit_bytes from in and writes units * out_words * 4 bytes to out (both device memory, 16-byte
// aligned in), on stream (NULL: the default stream). unit_bytes = seg_bytes * {1, 2, 4, 8}; seg_bytes one of
// 64, 128, 256, 512. Returns 0, or -1 for arguments out of range or a failed launch.
extern "C" int pitch_calib_stream(const void* in, void* out, uint64_t units, uint32_t unit_bytes,
                                  uint32_t out_words, uint32_t seg_bytes, uint32_t workgroups,
                                  uint32_t nontemporal, void* stream) {
  using namespace pitch_calib;
  if (!in || !out || units == 0 || seg_bytes == 0 || unit_bytes % seg_bytes != 0 || ((uintptr_t)in & 15u) ||
      ((uintptr_t)out & 3u))
    return -1;
  const uint32_t cpl = unit_bytes / seg_bytes;
  const bool nt = nontemporal != 0;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (seg_bytes) {
    case 64: e = launch_cpl<4>(cpl, in, out, units, out_words, workgroups, nt, s); break;
    case 128: e = launch_cpl<8>(cpl, in, out, units, out_words, workgroups, nt, s); break;
    case 256: e = launch_cpl<16>(cpl, in, out, units, out_words, workgroups, nt, s); break;
    case 512: e = launch_cpl<32>(cpl, in, out, units, out_words, workgroups, nt, s); break;
    default: return -1;
  }
  return e == hipSuccess ? 0 : -1;
}
