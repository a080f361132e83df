// Measurement kernels for bench.py (libpitch_calib.so): not part of the codec, and not declared in
// include/pitch_amd.h.
//
// calib_stream moves the bytes an encoder moves, with no arithmetic between its loads and its stores: each
// unit (one vector, or one token row of a key cache) is unit_bytes read and out_words 4-byte words written.
// The loads follow a chosen access shape, so the measured rate is the ceiling of that shape at that footprint:
// - seg_bytes: the contiguous piece of one unit that one load instruction reads per unit. A wave's load
//   instruction covers 64 * 16 / seg_bytes units, seg_bytes each; a unit takes unit_bytes / seg_bytes
//   instructions, and a wave takes 16 units per block (as the staged encoder and the streaming decoder do). The staged encoders read 64-byte pieces at d = 64 and 128-byte pieces at d = 128 (four or
//   eight lanes of 16 bytes per vector per instruction); the KIVI encoder reads 128-byte row pieces.
// - workgroups: the grid. Non-zero: a persistent grid of that many 256-thread workgroups striding over the
//   units (the encoders run 3 workgroups per CU); zero: one block of units per workgroup, all in one launch.
// - nontemporal: non-temporal loads and stores (the encoders use them), or cached ones.
// The stores are coalesced: a wave's units write one contiguous run of words, as the encoders' codes do.
// Every lane's loaded words feed a value that is compared before the stores, so the compiler keeps every load.
// calib_store is the decoders' mirror image (small coalesced reads, large stores in a chosen shape).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace pitch_calib {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr uint32_t kNever = 0x9E3779B9u;  // a fold value that stores to word 0 (keeps the loads live)

// A wave takes kWaveUnits units per block (the staged encoder's and the streaming decoder's 16 vectors per wave
// iteration): G = kWaveUnits / UPW load (or store) instructions per piece of a unit, UPW = 64 / L units each.
constexpr int kWaveUnits = 16;

// L lanes read one unit's seg piece (L * 16 bytes); CPL pieces per unit (unit = L * CPL * 16 bytes).
template <int L, int CPL, bool NT>
__global__ __launch_bounds__(kBlock) void calib_stream(const u32x4* __restrict__ in, uint32_t* __restrict__ out,
                                                       uint64_t units, uint32_t out_words, uint64_t grid_blocks) {
  constexpr int UPW = 64 / L;  // units per wave and instruction
  constexpr int G = kWaveUnits / UPW;
  static_assert(G >= 1 && G * UPW == kWaveUnits, "wave block");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ul = lane / L, pl = lane % L;
  const uint64_t wblocks = (units + kWaveUnits - 1) / kWaveUnits;
  for (uint64_t wb = (uint64_t)blockIdx.x * (kBlock / 64) + wave; wb < wblocks; wb += grid_blocks * (kBlock / 64)) {
    u32x4 c[G][CPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      uint64_t u = wb * kWaveUnits + g * UPW + ul;
      if (u >= units) u = units - 1;  // the last wave block re-reads the last unit
      const u32x4* src = in + u * (uint64_t)(L * CPL) + pl;
#pragma unroll
      for (int i = 0; i < CPL; ++i) c[g][i] = NT ? __builtin_nontemporal_load(src + i * L) : src[i * L];
    }
    uint32_t acc = 0;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < CPL; ++i) acc ^= c[g][i].x ^ c[g][i].y ^ c[g][i].z ^ c[g][i].w;
    if (acc == kNever) out[0] = acc;
    // the wave's units own one contiguous run of kWaveUnits * out_words words (as an encoder's codes): lane l
    // writes words l, l + 64, ... of it, up to the last unit's end
    const uint64_t w0 = wb * kWaveUnits * (uint64_t)out_words;
    const uint64_t wend = units * (uint64_t)out_words;
    const uint64_t run = (uint64_t)kWaveUnits * out_words;
    for (uint64_t j = lane; j < run && w0 + j < wend; j += 64) {
      if constexpr (NT) __builtin_nontemporal_store(acc + (uint32_t)j, out + w0 + j);
      else out[w0 + j] = acc + (uint32_t)j;
    }
  }
}

template <int L, int CPL>
hipError_t launch(const void* in, void* out, uint64_t units, uint32_t out_words, uint32_t workgroups, bool nt,
                  hipStream_t s) {
  const uint64_t wblocks = (units + kWaveUnits - 1) / kWaveUnits;
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

// The decoders' mirror image: each unit reads in_words 4-byte words (a wave's units one contiguous run, as the
// decoders' codes) and writes unit_bytes in pieces of L * 16 bytes per store instruction (CPL instructions per
// piece group). Workgroup blocks first_block on; each workgroup takes wave blocks blockIdx.x * 4 + wave of them,
// then strides by grid_blocks * 4 (a grid of one block per workgroup runs none twice).
template <int L, int CPL, bool NT>
__global__ __launch_bounds__(kBlock) void calib_store(const uint32_t* __restrict__ in, u32x4* __restrict__ out,
                                                      uint64_t units, uint32_t in_words, uint64_t first_block,
                                                      uint64_t grid_blocks) {
  constexpr int UPW = 64 / L;
  constexpr int G = kWaveUnits / UPW;
  static_assert(G >= 1 && G * UPW == kWaveUnits, "wave block");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ul = lane / L, pl = lane % L;
  const uint64_t wblocks = (units + kWaveUnits - 1) / kWaveUnits;
  for (uint64_t wb = (first_block + blockIdx.x) * (kBlock / 64) + wave; wb < wblocks;
       wb += grid_blocks * (kBlock / 64)) {
    const uint64_t w0 = wb * kWaveUnits * (uint64_t)in_words;
    const uint64_t wend = units * (uint64_t)in_words;
    const uint64_t run = (uint64_t)kWaveUnits * in_words;
    uint32_t acc = (uint32_t)wb;
    for (uint64_t j = lane; j < run && w0 + j < wend; j += 64)
      acc ^= NT ? __builtin_nontemporal_load(in + w0 + j) : in[w0 + j];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      uint64_t u = wb * kWaveUnits + g * UPW + ul;
      if (u >= units) u = units - 1;  // the last wave block rewrites the last unit with the same values
      u32x4* dst = out + u * (uint64_t)(L * CPL) + pl;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const u32x4 v = {acc, acc + 1u, acc + 2u, (uint32_t)i};
        if constexpr (NT) __builtin_nontemporal_store(v, dst + i * L);
        else dst[i * L] = v;
      }
    }
  }
}

template <int L, int CPL>
hipError_t launch_store(const void* in, void* out, uint64_t units, uint32_t in_words, uint32_t mode,
                        uint32_t workgroups, bool nt, hipStream_t s) {
  const uint64_t wblocks = (units + kWaveUnits - 1) / kWaveUnits;
  const uint64_t blocks = (wblocks + kBlock / 64 - 1) / (kBlock / 64);  // workgroup blocks
  auto go = [&](uint64_t grid, uint64_t first, uint64_t stride_blocks) {
    if (nt)
      hipLaunchKernelGGL((calib_store<L, CPL, true>), dim3((uint32_t)grid), dim3(kBlock), 0, s,
                         (const uint32_t*)in, (u32x4*)out, units, in_words, first, stride_blocks);
    else
      hipLaunchKernelGGL((calib_store<L, CPL, false>), dim3((uint32_t)grid), dim3(kBlock), 0, s,
                         (const uint32_t*)in, (u32x4*)out, units, in_words, first, stride_blocks);
  };
  if (mode == 0) {  // persistent: workgroups striding over every block
    if (workgroups == 0) return hipErrorInvalidValue;
    go(workgroups, 0, workgroups);
  } else if (mode == 1) {  // one launch, one block per workgroup
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    go(blocks, 0, blocks);
  } else {  // launches of `workgroups` workgroups, one block each
    if (workgroups == 0) return hipErrorInvalidValue;
    for (uint64_t b0 = 0; b0 < blocks; b0 += workgroups)
      go(blocks - b0 < workgroups ? blocks - b0 : workgroups, b0, blocks);
  }
  return hipGetLastError();
}

template <int L>
hipError_t launch_store_cpl(uint32_t cpl, const void* in, void* out, uint64_t units, uint32_t in_words,
                            uint32_t mode, uint32_t workgroups, bool nt, hipStream_t s) {
  switch (cpl) {
    case 1: return launch_store<L, 1>(in, out, units, in_words, mode, workgroups, nt, s);
    case 2: return launch_store<L, 2>(in, out, units, in_words, mode, workgroups, nt, s);
    case 4: return launch_store<L, 4>(in, out, units, in_words, mode, workgroups, nt, s);
    case 8: return launch_store<L, 8>(in, out, units, in_words, mode, workgroups, nt, s);
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

// Decoder-shaped stream: reads units * in_words * 4 bytes from in (a wave's units one contiguous run) and writes
// units * unit_bytes to out (16-byte aligned) in pieces of seg_bytes (64, 128, 256 or 512; unit_bytes = seg_bytes
// * {1, 2, 4, 8}). mode 0: one persistent launch of `workgroups` workgroups; 1: one launch of one block per
// workgroup; 2: launches of `workgroups` workgroups, one block each (the streaming decoder's shape). Returns 0, or
// -1 for arguments out of range or a failed launch.
extern "C" int pitch_calib_stream_store(const void* in, void* out, uint64_t units, uint32_t unit_bytes,
                                        uint32_t in_words, uint32_t seg_bytes, uint32_t mode, uint32_t workgroups,
                                        uint32_t nontemporal, void* stream) {
  using namespace pitch_calib;
  if (!in || !out || units == 0 || seg_bytes == 0 || unit_bytes % seg_bytes != 0 || mode > 2 ||
      ((uintptr_t)out & 15u) || ((uintptr_t)in & 3u))
    return -1;
  const uint32_t cpl = unit_bytes / seg_bytes;
  const bool nt = nontemporal != 0;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (seg_bytes) {
    case 64: e = launch_store_cpl<4>(cpl, in, out, units, in_words, mode, workgroups, nt, s); break;
    case 128: e = launch_store_cpl<8>(cpl, in, out, units, in_words, mode, workgroups, nt, s); break;
    case 256: e = launch_store_cpl<16>(cpl, in, out, units, in_words, mode, workgroups, nt, s); break;
    case 512: e = launch_store_cpl<32>(cpl, in, out, units, in_words, mode, workgroups, nt, s); break;
    default: return -1;
  }
  return e == hipSuccess ? 0 : -1;
}
