// Per-channel (KIVI-style) key encode/decode for one element type of the uncompressed keys (PITCH_IO: 0 float32,
// 1 float16, 2 bfloat16; 16-bit keys are widened to float32 exactly, decoded float32 values are rounded to
// nearest even). The generic pack/unpack kernels are built with PITCH_IO = 0.
//
// Semantics follow reference/pitch_reference.py:145-174 bit for bit: per group of G tokens and per channel,
// float32 min and max rounded to fp16 (round to nearest even), step = (f32(hi16) - f32(lo16)) / (2^b - 1)
// with 0 -> 1, code = clip(floor((x - lo) / step + 0.5), 0, 2^b - 1), all in float32 with correctly
// rounded division; decode x = f32(code) * step + lo as two roundings (no fused multiply-add; the library
// is built with -ffp-contract=off). The Metal kernels they replace (PITCHKernels.metal:262-325) read each
// group twice and pack one token per barrier; here a workgroup loads a group once, keeps up to kMaxR
// tokens per thread in registers between the range pass and the quantise pass, and packs codes from LDS.
#include <hip/hip_fp16.h>

#include "pitch_device.h"

#ifndef PITCH_IO
#define PITCH_IO 0
#endif

namespace pitch {
namespace {

constexpr int kMaxR = 8;           // tokens per thread held in registers between the two passes
constexpr int kStageBytes = 8192;  // LDS staging for one tile of codes (one byte per code)
constexpr int kDecR = 4;           // tokens per thread per decode iteration

__device__ __forceinline__ uint16_t f2h_bits(float x) { return __half_as_ushort(__float2half_rn(x)); }
__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }

// Groups of G tokens in a call of count tokens, in 64 bits: count may be up to 2^32 - 1 and count + G - 1 would
// wrap in 32 bits.
__device__ __forceinline__ uint32_t group_count(uint32_t count, uint32_t G) {
  return (uint32_t)(((uint64_t)count + G - 1u) / G);
}

__device__ __forceinline__ float kivi_step(float lo, float hi, float levels) {
  const float s = (hi - lo) / levels;
  return s == 0.0f ? 1.0f : s;
}

__device__ __forceinline__ uint32_t kivi_code(float x, float base, float step, float levels) {
  const float q = floorf((x - base) / step + 0.5f);
  return (uint32_t)fminf(fmaxf(q, 0.0f), levels);
}

// Packs token rows of `dim` one-byte codes (stage[tok * dim + i]) into words. Word wi of a row holds the
// bits [32*wi, 32*wi + 32) of the row's code stream (reference/pitch_reference.py:68-78).
template <int B>
__device__ __forceinline__ void pack_rows(const uint8_t* stage, uint32_t ntok, uint32_t dim, uint32_t nwords,
                                          uint32_t* dst) {
  if ((dim & 31u) == 0u) {
    // rows split into groups of 32 codes that pack into exactly B words each
    const uint32_t gpr = dim >> 5;
    const uint32_t ng = ntok * gpr;
    for (uint32_t g = threadIdx.x; g < ng; g += kBlock) {
      const uint32_t tok = g / gpr, gi = g - tok * gpr;
      const uint4* q = (const uint4*)(stage + tok * dim + 32u * gi);
      const uint4 q0 = q[0], q1 = q[1];
      const uint32_t bytes[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      uint32_t w[B];
      pack32<B>(bytes, w);
      store_words<B>(dst + (uint64_t)tok * nwords + gi * B, w);
    }
  } else {
    const uint32_t nw = ntok * nwords;
    for (uint32_t w = threadIdx.x; w < nw; w += kBlock) {
      const uint32_t tok = w / nwords, wi = w - tok * nwords;
      const uint8_t* row = stage + tok * dim;
      uint32_t word = 0u;
      for (uint32_t i = (32u * wi) / B; i < dim; ++i) {
        const int s = (int)(i * B) - (int)(32u * wi);
        if (s >= 32) break;
        const uint32_t c = row[i];
        word |= s >= 0 ? (c << s) : (c >> (-s));
      }
      dst[(uint64_t)tok * nwords + wi] = word;
    }
  }
}

// ------------------------------------------------------------------------------------------- encode
// dim % 4 == 0: thread (phase pp, column chunk col) owns channels [4col, 4col+4) of tokens pp, pp+P, ...
template <int B, int IO>
__global__ __launch_bounds__(kBlock) void chan_encode4(ChanArgs p) {
  const float levels = (float)((1 << B) - 1);
  __shared__ float4 s_lo[kBlock], s_hi[kBlock];
  __shared__ float s_base[1024], s_step[1024];
  __shared__ __attribute__((aligned(16))) uint8_t s_stage[kStageBytes];

  const uint32_t dim = p.dim, C = dim >> 2, P = kBlock / C;
  const uint32_t tid = threadIdx.x, pp = tid / C, col = tid - pp * C;
  const bool active = pp < P;
  const uint32_t TT = min(P * kMaxR, (uint32_t)kStageBytes / dim);  // tokens per packing tile
  const uint32_t groups = group_count(p.count, p.group);

  for (uint64_t g = blockIdx.x; g < groups; g += gridDim.x) {  // 64-bit: g + gridDim.x must not wrap
    const uint32_t first = (uint32_t)(g * p.group);
    const uint32_t n = min(p.group, p.count - first);
    const uint64_t src = (uint64_t)first * dim + 4u * col;  // element index of this thread's first channel

    // pass 1: channel minima and maxima over the group
    float4 lo = make_float4(__builtin_inff(), __builtin_inff(), __builtin_inff(), __builtin_inff());
    float4 hi = make_float4(-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff());
    float4 cache[kMaxR];
#pragma unroll
    for (int i = 0; i < kMaxR; ++i) {
      const uint32_t tk = pp + i * P;
      if (active && tk < n) {
        float v[4];
        load_elems<IO, 4>(p.in, src + (uint64_t)tk * dim, v);
        const float4 x = make_float4(v[0], v[1], v[2], v[3]);
        cache[i] = x;
        lo = make_float4(fminf(lo.x, x.x), fminf(lo.y, x.y), fminf(lo.z, x.z), fminf(lo.w, x.w));
        hi = make_float4(fmaxf(hi.x, x.x), fmaxf(hi.y, x.y), fmaxf(hi.z, x.z), fmaxf(hi.w, x.w));
      }
    }
    for (uint32_t tk = pp + kMaxR * P; active && tk < n; tk += P) {
      float v[4];
      load_elems<IO, 4>(p.in, src + (uint64_t)tk * dim, v);
      const float4 x = make_float4(v[0], v[1], v[2], v[3]);
      lo = make_float4(fminf(lo.x, x.x), fminf(lo.y, x.y), fminf(lo.z, x.z), fminf(lo.w, x.w));
      hi = make_float4(fmaxf(hi.x, x.x), fmaxf(hi.y, x.y), fmaxf(hi.z, x.z), fmaxf(hi.w, x.w));
    }
    s_lo[tid] = lo;
    s_hi[tid] = hi;
    __syncthreads();
    if (tid < C) {
      float4 l = s_lo[tid], h = s_hi[tid];
      for (uint32_t q = 1; q < P; ++q) {
        const float4 a = s_lo[q * C + tid], b = s_hi[q * C + tid];
        l = make_float4(fminf(l.x, a.x), fminf(l.y, a.y), fminf(l.z, a.z), fminf(l.w, a.w));
        h = make_float4(fmaxf(h.x, b.x), fmaxf(h.y, b.y), fmaxf(h.z, b.z), fmaxf(h.w, b.w));
      }
      float lv[4] = {l.x, l.y, l.z, l.w}, hv[4] = {h.x, h.y, h.z, h.w};
      // an extreme of zero takes the sign of the channel's last zero in token order (numpy's min / max keep the
      // last of equal values); rare, so the channel is scanned again
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (lv[r] == 0.0f || hv[r] == 0.0f) {
          float zs = 0.0f;
          for (uint32_t tk = 0; tk < n; ++tk) {
            float v[1];
            load_elems<IO, 1>(p.in, (uint64_t)first * dim + (uint64_t)tk * dim + 4u * tid + r, v);
            if (v[0] == 0.0f) zs = v[0];
          }
          if (lv[r] == 0.0f) lv[r] = zs;
          if (hv[r] == 0.0f) hv[r] = zs;
        }
      }
      uint16_t l16[4], h16[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        l16[r] = f2h_bits(lv[r]);
        h16[r] = f2h_bits(hv[r]);
        const float b0 = h2f(l16[r]);
        s_base[4 * tid + r] = b0;
        s_step[4 * tid + r] = kivi_step(b0, h2f(h16[r]), levels);
      }
      uint16_t* rg = p.ranges_out + (uint64_t)g * 2u * dim + 4u * tid;
      *(u32x2*)rg = u32x2{(uint32_t)l16[0] | ((uint32_t)l16[1] << 16), (uint32_t)l16[2] | ((uint32_t)l16[3] << 16)};
      *(u32x2*)(rg + dim) =
          u32x2{(uint32_t)h16[0] | ((uint32_t)h16[1] << 16), (uint32_t)h16[2] | ((uint32_t)h16[3] << 16)};
    }
    __syncthreads();

    // pass 2: quantise tile by tile, stage one byte per code, pack rows
    float bs[4] = {0.f, 0.f, 0.f, 0.f}, st[4] = {1.f, 1.f, 1.f, 1.f};
    if (active) {
#pragma unroll
      for (int r = 0; r < 4; ++r) { bs[r] = s_base[4 * col + r]; st[r] = s_step[4 * col + r]; }
    }
    for (uint32_t tb = 0; tb < n; tb += TT) {
      const uint32_t nt = min(TT, n - tb);
      for (uint32_t i = 0; i * P < nt; ++i) {
        const uint32_t tk = tb + pp + i * P;
        if (active && tk < tb + nt) {
          float4 x;
          bool cached = false;
#pragma unroll
          for (int j = 0; j < kMaxR; ++j) {
            if (tb == 0 && (uint32_t)j == i) { x = cache[j]; cached = true; }
          }
          if (!cached) {
            float v[4];
            load_elems<IO, 4>(p.in, src + (uint64_t)tk * dim, v);
            x = make_float4(v[0], v[1], v[2], v[3]);
          }
          const uint32_t c = kivi_code(x.x, bs[0], st[0], levels) | (kivi_code(x.y, bs[1], st[1], levels) << 8) |
                             (kivi_code(x.z, bs[2], st[2], levels) << 16) |
                             (kivi_code(x.w, bs[3], st[3], levels) << 24);
          *(uint32_t*)(s_stage + (tk - tb) * dim + 4u * col) = c;
        }
      }
      __syncthreads();
      pack_rows<B>(s_stage, nt, dim, p.nwords, p.codes_out + (uint64_t)(first + tb) * p.nwords);
      __syncthreads();
    }
  }
}

// ------------------------------------------------------------------------------------------- encode, G <= 64
// One wave per (group, slab of 64 channels), four independent waves per workgroup, no workgroup barriers.
// Lane (r, c) = (lane / 16, lane % 16) holds channels 4c .. 4c+3 of the slab for tokens r, r + 4, ..., r + 60
// of the group, so each load instruction reads four token rows of 256 bytes. The channel minima and maxima
// are reduced across the four token phases with two lane exchanges; every lane then knows the fp16 range of
// its channels. Codes are staged as bytes in the wave's LDS slice and packed 32 at a time.
//
// Quantiser: the reference's t = RN(RN((x - lo) / step) + 0.5) (pitch_reference.py:157, float32) exactly,
// without a division per element. With inv = RN(1 / step) (one correctly rounded division per channel),
// q0 = RN(a * inv) is within one ulp of a / step, the residual r = a - q0 * step is exact in one fma, and
// q0 + r * inv rounded once is RN(a / step) (Markstein's theorem for a correctly rounded reciprocal). The
// step itself, RN((hi - lo) / (2^B - 1)), is obtained the same way with the constant RN(1 / (2^B - 1)).
// Outside the theorem's range nothing decides a code: a step of +inf (a range end beyond fp16) is clamped to
// FLT_MAX in the residual so that a finite a gives q = 0 as a / inf does, and only a subnormal quotient
// (|a / step| < 2^-126, whose code is 0 either way) may differ from RN(a / step).
#ifndef PITCH_KIVI_WAVES
#define PITCH_KIVI_WAVES 3  // waves per SIMD the per-channel encoder's register budget allows
#endif
#ifndef PITCH_KIVI_DEC_SLAB
#define PITCH_KIVI_DEC_SLAB 64
#endif
constexpr int kSlab = PITCH_KIVI_DEC_SLAB;  // channels per wave of the decoder (long calls)
#ifndef PITCH_KIVI_DEC_SLAB32
#define PITCH_KIVI_DEC_SLAB32 1  // 1: 32-channel decoder slabs for float32 calls of at most PITCH_KIVI_DEC_SLAB32_MAX
#endif                           // (group, 64-channel) items
#ifndef PITCH_KIVI_DEC_SLAB32_MAX
#define PITCH_KIVI_DEC_SLAB32_MAX 32768
#endif
constexpr int kGroupMaxW = 64;   // largest group the wave encoder takes
// Calls of the wave encoder and decoder longer than this many rounds (grid-stride iterations per workgroup) are
// issued as several launches of this many rounds. At a 17 GB footprint (config 5 keys: 33.5M tokens, d = 128) a
// single persistent launch reaches 4.4 TB/s encoding and 4.9 TB/s decoding; launches of 2 rounds reach 5.3 and
// 5.35 TB/s, of 1 round 5.0 and 5.4 (the same box, one run: encode 5.0 / 5.4, decode 5.42 / 5.36 TB/s for 1 / 2
// rounds). A launch boundary brings every workgroup back in step; in one long launch they drift apart, and the
// reads of some interleave with the writes of others at the memory (a probe kernel with the decoder's read/write mix
// showed the same gain from short launches). Calls of up to this many rounds keep one launch.
constexpr uint64_t kChanSliceRoundsEnc = 2;
constexpr uint64_t kChanSliceRoundsDec = 1;
#ifndef PITCH_KIVI_DEC_CPL8
// 16-bit decodes at B <= 4 of whole 64-channel slabs: eight channels per lane from this many (group, slab) items
// (d = 64, b = 4, float16 and bfloat16, two interleaved repeats: 4M tokens 57.2-58.3 -> 59.0-60.6 % of peak, 1M
// 54.8-57.3 -> 55.1-57.9 %, but config 3's 262K tokens 49.2-49.7 -> 47.9-48.5 %: each lane's range set-up doubles)
#define PITCH_KIVI_DEC_CPL8 1
#endif
#ifndef PITCH_KIVI_DEC_CPL8_MIN_ITEMS
#define PITCH_KIVI_DEC_CPL8_MIN_ITEMS 16384u
#endif
#ifndef PITCH_KIVI_DEC_NTS
// The wave decoder writes keys with non-temporal stores (cached stores measured 7.5 % slower at config 5's keys and
// 23 % slower at config 3's, two repeats each).
#define PITCH_KIVI_DEC_NTS 1
#endif
// Long float32 calls of the wave decoder and encoder run one launch of one work item per wave, with far more
// workgroups than the CUs hold, and with fewer of them resident per CU than the kernels' registers allow: dynamic
// LDS (lds_cap_bytes) holds the decoder at 4 and the encoder at 2 workgroups per CU. Config 5's keys (33.5M tokens,
// d = 128, b = 4; interleaved repeats on one box, identical bytes): decode 5.40-5.43 TB/s in launches of one round
// at the decoder's full 8 per CU; one launch at 3 / 4 / 5 / 6 per CU 5.35-5.41 / 5.81-5.83 / 5.64-5.67 / 5.37-5.39;
// encode 5.51-5.52 at its full 4 per CU, 5.39-5.41 at 3, 5.70-5.74 at 2. Shorter calls, d = 128, b = 4 (rounds
// at full occupancy; two repeats, identical bytes): decode 1M tokens (8 rounds of 32-channel slabs) 6.06 -> 6.35-6.40,
// 2M (8 rounds) 6.50 -> 6.38-6.43, 4M (16 rounds) 5.45-5.48 -> 6.04-6.11; encode 1M (11 rounds) 5.34-5.38 ->
// 4.99-5.01, 2M (16 rounds) 5.63-5.67 -> 5.98-6.01, config 3 (8 x 32768 tokens at d = 64, 2-4 rounds) 5.25-5.34 ->
// 4.24-4.29. Hence one launch from 8 rounds for the decoder and from 16 for the encoder. The encoder's 32-channel slabs
// (calls of at most 32,768 (group, 64-channel) items) run one launch at their full 4 per CU from 4 rounds: d = 64 at
// 2^19 - 2^21 tokens 65-67 -> 70.5-73.3 % of peak, d = 128 at 2^18 - 2^20 65-66 -> 72.1-72.5 % (two repeats, identical
// bytes; at 2 per CU 53-63 %, at 3 per CU 62-71 %); at 2 rounds (config 3) the balanced persistent grid stays (65.5
// against 64.5 %), and the 64-channel slabs of longer calls keep 2 per CU from 16 rounds (71-73 % against 70 % at 4).
#ifndef PITCH_KIVI_DEC_ONE_LAUNCH
#define PITCH_KIVI_DEC_ONE_LAUNCH 1  // float32 decode calls of PITCH_KIVI_DEC_MIN_ROUNDS+ rounds: one launch
#endif
#ifndef PITCH_KIVI_DEC_MIN_ROUNDS
#define PITCH_KIVI_DEC_MIN_ROUNDS 8  // resident rounds (at full occupancy) from which the one-launch decode runs
#endif
#ifndef PITCH_KIVI_DEC_WG_PER_CU
#define PITCH_KIVI_DEC_WG_PER_CU 4  // resident decoder workgroups per CU in the one-launch mode (0: no cap)
#endif
#ifndef PITCH_KIVI_ENC_WG_PER_CU
#define PITCH_KIVI_ENC_WG_PER_CU 2  // resident encoder workgroups per CU in the one-launch mode (0: no cap)
#endif
#ifndef PITCH_KIVI_ENC_ONE_LAUNCH
#define PITCH_KIVI_ENC_ONE_LAUNCH 1  // float32 encode calls of PITCH_KIVI_ENC_MIN_ROUNDS+ rounds: one launch
#endif
#ifndef PITCH_KIVI_ENC_MIN_ROUNDS
#define PITCH_KIVI_ENC_MIN_ROUNDS 16  // resident rounds (balanced grid) from which the one-launch encode runs
#endif
#ifndef PITCH_KIVI_ENC_MIN_ROUNDS32
#define PITCH_KIVI_ENC_MIN_ROUNDS32 4  // the same for 32-channel slabs
#endif
#ifndef PITCH_KIVI_ENC_WG_PER_CU32
#define PITCH_KIVI_ENC_WG_PER_CU32 0  // resident workgroups per CU of 32-channel one-launch encodes (0: no cap)
#endif
#ifndef PITCH_KIVI_NT
#define PITCH_KIVI_NT 1  // the wave encoder reads keys with non-temporal loads
#endif
#ifndef PITCH_KIVI_NTS
// Non-temporal stores of codes and ranges. Off: a 32-channel slab writes half of each token's code row and
// of each range row, and cached stores let L2 merge the halves of neighbouring slabs into whole lines (with
// non-temporal stores the encoder wrote 1.5x its algorithmic bytes)
#define PITCH_KIVI_NTS 0
#endif
#ifndef PITCH_KIVI_DP
#define PITCH_KIVI_DP 1  // direct packing in the wave encoder where the bit width and row width allow it
#endif
#ifndef PITCH_KIVI_BALANCE
#define PITCH_KIVI_BALANCE 1  // 1: the float32 wave encoder asks for balanced rounds
#endif
#ifndef PITCH_KIVI_SLAB
#define PITCH_KIVI_SLAB 0        // encoder slab width: 0 = chosen per call, else 32 or 64 channels
#endif

// SW = 64: lane (r, c) = (lane / 16, lane % 16), tokens r, r + 4, ... (16 per lane); SW = 32: lane
// (lane / 8, lane % 8), tokens r, r + 8, ... (8 per lane), twice the work items and half the registers.
// DP (direct packing; B = 2, 4 or 8 and a row width that is a multiple of SW): lane c's four codes of a token
// are the byte-aligned bit-field [4 B c, 4 B c + 4 B) of the row's packed code stream, so the lane packs them
// in registers and writes B / 2 bytes of packed row to LDS; the stores then copy packed rows.
template <int B, int IO, int SW, bool DP>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(PITCH_KIVI_WAVES))) void chan_encode_w(ChanArgs p) {
  static_assert(!DP || B == 2 || B == 4 || B == 8, "direct packing needs byte-aligned lane fields");
  constexpr int QW = SW / 4;           // lanes per token row
  constexpr int RPI = 64 / QW;         // token rows per load instruction
  constexpr int TPL = kGroupMaxW / RPI;  // tokens per lane
  const float levels = (float)((1 << B) - 1);
  __shared__ __attribute__((aligned(16))) uint8_t s_stage_all[kBlock / 64][kGroupMaxW * SW];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint8_t* s_stage = s_stage_all[wid];
  const int r = lane / QW, c = lane % QW;
  const uint32_t dim = p.dim, G = p.group;
  const uint32_t slabs = (dim + SW - 1) / SW;
  const uint32_t groups = group_count(p.count, G);
  const uint64_t items = (uint64_t)groups * slabs;
  const uint64_t waves = (uint64_t)gridDim.x * (kBlock / 64);

  for (uint64_t it = (uint64_t)blockIdx.x * (kBlock / 64) + wid; it < items; it += waves) {
    const uint32_t g = (uint32_t)(it / slabs), sl = (uint32_t)(it - (uint64_t)g * slabs);
    const uint32_t first = g * G, n = min(G, p.count - first);
    const uint32_t ch0 = sl * SW, cw = min((uint32_t)SW, dim - ch0);  // cw is a multiple of 4
    const bool cact = 4u * c < cw;
    const uint64_t src = (uint64_t)first * dim + ch0 + (cact ? 4u * c : 0u);  // element index

    // loads: rows past the group's end re-read its last row (no effect on the range). In a group of all
    // kGroupMaxW rows no row is clamped: each load is then a wave-uniform row base plus the lane's 32-bit byte
    // offset, with no per-lane 64-bit address arithmetic.
    float4 x[TPL];
    if (n == (uint32_t)kGroupMaxW) {
      constexpr uint32_t ES = IO == 0 ? 4u : 2u;  // bytes per key element
      const char* gbase = (const char*)p.in + ((uint64_t)first * dim + ch0) * ES;
      const uint32_t loff = (r * dim + (cact ? 4u * c : 0u)) * ES;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        const char* row = gbase + (uint64_t)(RPI * i) * dim * ES;
        float v[4];
        if constexpr (PITCH_KIVI_NT) load4_nt<IO>(row + loff, 0, v);
        else load_elems<IO, 4>(row + loff, 0, v);
        x[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        const uint32_t tk = r + (uint32_t)RPI * i;
        float v[4];
        if constexpr (PITCH_KIVI_NT) load4_nt<IO>(p.in, src + (uint64_t)(tk < n ? tk : n - 1) * dim, v);
        else load_elems<IO, 4>(p.in, src + (uint64_t)(tk < n ? tk : n - 1) * dim, v);
        x[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
    // minima and maxima with the hardware's min3 / max3 / min / max (no canonicalising of the loaded and
    // exchanged values, which fminf / fmaxf would add)
    float l[4], h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      auto e = [&](int i) { return k == 0 ? x[i].x : k == 1 ? x[i].y : k == 2 ? x[i].z : x[i].w; };
      float mn = e(0), mx = e(0);
      int i = 1;
#pragma unroll
      for (; i + 1 < TPL; i += 2) {
        mn = fmin3_hw(mn, e(i), e(i + 1));
        mx = fmax3_hw(mx, e(i), e(i + 1));
      }
      if (i < TPL) {
        mn = fmin_hw(mn, e(i));
        mx = fmax_hw(mx, e(i));
      }
      l[k] = mn;
      h[k] = mx;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int off = QW; off < 64; off <<= 1) {
        l[k] = fmin_hw(l[k], __shfl_xor(l[k], off));
        h[k] = fmax_hw(h[k], __shfl_xor(h[k], off));
      }
    }
    // an extreme of zero takes the sign of the channel's last zero in token order, as numpy's min / max keep the
    // last of equal values (rare: the lanes of a channel take this branch together, and exchange only among
    // themselves)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (l[k] == 0.0f || h[k] == 0.0f) {
        int z = -1;
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
          const uint32_t tk = r + (uint32_t)RPI * i;
          const float xv = k == 0 ? x[i].x : k == 1 ? x[i].y : k == 2 ? x[i].z : x[i].w;
          if (tk < n && xv == 0.0f) z = max(z, (int)(2u * tk + (__float_as_uint(xv) >> 31)));
        }
#pragma unroll
        for (int off = QW; off < 64; off <<= 1) z = max(z, __shfl_xor(z, off));
        const float zs = (z & 1) ? -0.0f : 0.0f;
        if (l[k] == 0.0f) l[k] = zs;
        if (h[k] == 0.0f) h[k] = zs;
      }
    }
    uint16_t l16[4], h16[4];
    float bs[4], stc[4], inv[4];
    constexpr float kInvLevels = 1.0f / (float)((1 << B) - 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      l16[k] = f2h_bits(l[k]);
      h16[k] = f2h_bits(h[k]);
      bs[k] = h2f(l16[k]);
      const float d = h2f(h16[k]) - bs[k];
      const float s0 = d * kInvLevels;
      const float sq = __builtin_fmaf(__builtin_fmaf(-s0, levels, d), kInvLevels, s0);  // RN(d / levels)
      const float st = sq == 0.0f ? 1.0f : sq;                                            // kivi_step
      inv[k] = rcp_rn(st);
      stc[k] = __builtin_fminf(st, 0x1.fffffep127f);
    }
    if (r == 0 && cact) {
      uint16_t* rg = p.ranges_out + (uint64_t)g * 2u * dim + ch0 + 4u * c;
      store_v((u32x2*)rg, u32x2{(uint32_t)l16[0] | ((uint32_t)l16[1] << 16), (uint32_t)l16[2] | ((uint32_t)l16[3] << 16)},
              PITCH_KIVI_NTS);
      store_v((u32x2*)(rg + dim),
              u32x2{(uint32_t)h16[0] | ((uint32_t)h16[1] << 16), (uint32_t)h16[2] | ((uint32_t)h16[3] << 16)},
              PITCH_KIVI_NTS);
    }
    // codes clip(floor((x - lo) / step + 0.5), 0, 2^B - 1) (pitch_reference.py:157-158), one byte each in LDS.
    // Rows past the group's end and channels past the slab's end are quantised and staged too (their slots
    // exist and are never packed), so the loop has no branches.
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const uint32_t tk = r + (uint32_t)RPI * i;
      const float xv[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
      uint32_t word = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = xv[k] - bs[k];
        const float q0 = a * inv[k];
        const float q = __builtin_fmaf(__builtin_fmaf(-q0, stc[k], a), inv[k], q0);  // RN(a / step)
        // clip(floor(q + 0.5), 0, 2^B - 1): q + 0.5 rounded to float32 as in the reference, then one flooring
        // convert and an integer med3
        const uint32_t t = (uint32_t)min(max(cvt_flr_i32(q + 0.5f), 0), (1 << B) - 1);
        if constexpr (DP && B < 8) word |= t << (B * k);           // packed field
        else word |= t << (8 * k);                                 // byte k
      }
      if constexpr (DP) {
        uint8_t* row = s_stage + tk * (SW * B / 8) + c * (B / 2);
        if constexpr (B == 2) *row = (uint8_t)word;
        else if constexpr (B == 4) *(uint16_t*)row = (uint16_t)word;
        else *(uint32_t*)row = word;
      } else {
        *(uint32_t*)(s_stage + tk * SW + 4u * c) = word;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // pack: the slab's codes of a token start at word ch0 * B / 32 of its row (ch0 is a multiple of 64)
    uint32_t* dst = p.codes_out + (uint64_t)first * p.nwords + ch0 * B / 32u;
    if constexpr (DP) {
      // packed rows of SW * B / 8 bytes in LDS, each the slab's part of a token row
      constexpr int RW = SW * B / 32;                 // words per packed LDS row
      constexpr int PW = RW >= 4 ? 4 : RW;            // words per copy
      constexpr uint32_t pr = RW / PW;  // copies per row (every slab is full: cw = SW)
      const uint32_t np = n * pr;
      for (uint32_t q = lane; q < np; q += 64) {
        const uint32_t tok = q / pr, pi = q - tok * pr;
        const uint32_t* src = (const uint32_t*)(s_stage + tok * (SW * B / 8)) + PW * pi;
        uint32_t* d = dst + (uint64_t)tok * p.nwords + PW * pi;
        if constexpr (PW == 4) store_v((u32x4*)d, *(const u32x4*)src, PITCH_KIVI_NTS);
        else if constexpr (PW == 2) store_v((u32x2*)d, *(const u32x2*)src, PITCH_KIVI_NTS);
        else store_v(d, *src, PITCH_KIVI_NTS);
      }
    } else if ((cw & 31u) == 0u) {
      const uint32_t gpr = cw >> 5, ng = n * gpr;  // 32-code groups per row, then in all
      for (uint32_t q = lane; q < ng; q += 64) {
        const uint32_t tok = q / gpr, gi = q - tok * gpr;
        const uint4* s4 = (const uint4*)(s_stage + tok * SW + 32u * gi);
        const uint4 q0 = s4[0], q1 = s4[1];
        const uint32_t bytes[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        uint32_t w[B];
        pack32<B>(bytes, w);
        if constexpr (PITCH_KIVI_NTS) store_words_nt<B>(dst + (uint64_t)tok * p.nwords + gi * B, w);
        else store_words<B>(dst + (uint64_t)tok * p.nwords + gi * B, w);
      }
    } else {
      // last, partial slab of a row whose width is not a multiple of 32: it ends the row
      const uint32_t wpr = p.nwords - ch0 * B / 32u, nw = n * wpr;
      for (uint32_t q = lane; q < nw; q += 64) {
        const uint32_t tok = q / wpr, wi = q - tok * wpr;
        const uint8_t* row = s_stage + tok * SW;
        uint32_t word = 0u;
        for (uint32_t i = (32u * wi) / B; i < cw; ++i) {
          const int sh = (int)(i * B) - (int)(32u * wi);
          if (sh >= 32) break;
          const uint32_t cd = row[i];
          word |= sh >= 0 ? (cd << sh) : (cd >> (-sh));
        }
        dst[(uint64_t)tok * p.nwords + wi] = word;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// dim % 4 != 0: one channel per thread for the ranges, one code per thread for quantisation
template <int B, int IO>
__global__ __launch_bounds__(kBlock) void chan_encode1(ChanArgs p) {
  const float levels = (float)((1 << B) - 1);
  __shared__ float s_base[1024], s_step[1024];
  __shared__ __attribute__((aligned(16))) uint8_t s_stage[kStageBytes];
  const uint32_t dim = p.dim, tid = threadIdx.x;
  const uint32_t TT = max(1u, (uint32_t)kStageBytes / dim);
  const uint32_t groups = group_count(p.count, p.group);
  for (uint64_t g = blockIdx.x; g < groups; g += gridDim.x) {  // 64-bit: g + gridDim.x must not wrap
    const uint32_t first = (uint32_t)(g * p.group);
    const uint32_t n = min(p.group, p.count - first);
    const uint64_t src = (uint64_t)first * dim;  // element index of the group's first token
    for (uint32_t ch = tid; ch < dim; ch += kBlock) {
      // in token order, keeping the later of equal values as numpy's min / max do (a zero extreme takes the sign
      // of the channel's last zero)
      float lo = __builtin_inff(), hi = -__builtin_inff();
      for (uint32_t tk = 0; tk < n; ++tk) {
        float xv[1];
        load_elems<IO, 1>(p.in, src + (uint64_t)tk * dim + ch, xv);
        const float x = xv[0];
        lo = lo < x ? lo : x;
        hi = hi > x ? hi : x;
      }
      const uint16_t l16 = f2h_bits(lo), h16 = f2h_bits(hi);
      p.ranges_out[(uint64_t)g * 2u * dim + ch] = l16;
      p.ranges_out[(uint64_t)g * 2u * dim + dim + ch] = h16;
      s_base[ch] = h2f(l16);
      s_step[ch] = kivi_step(h2f(l16), h2f(h16), levels);
    }
    __syncthreads();
    for (uint32_t tb = 0; tb < n; tb += TT) {
      const uint32_t nt = min(TT, n - tb);
      for (uint32_t it = tid; it < nt * dim; it += kBlock) {
        const uint32_t tok = it / dim, ch = it - tok * dim;
        float xv[1];
        load_elems<IO, 1>(p.in, src + (uint64_t)(tb + tok) * dim + ch, xv);
        s_stage[it] = (uint8_t)kivi_code(xv[0], s_base[ch], s_step[ch], levels);
      }
      __syncthreads();
      pack_rows<B>(s_stage, nt, dim, p.nwords, p.codes_out + (uint64_t)(first + tb) * p.nwords);
      __syncthreads();
    }
  }
}

// ------------------------------------------------------------------------------------------- decode
template <int B, int IO>
__global__ __launch_bounds__(kBlock) void chan_decode4(ChanArgs p) {
  const float levels = (float)((1 << B) - 1);
  constexpr uint32_t kMask = (1u << B) - 1u;
  const uint32_t dim = p.dim, C = dim >> 2, P = kBlock / C;
  const uint32_t tid = threadIdx.x, pp = tid / C, col = tid - pp * C;
  if (pp >= P) return;  // no barriers below
  const uint32_t TT = P * kDecR;
  const uint32_t pos = 4u * B * col, wi = pos >> 5, sh = pos & 31u;
  const bool straddle = sh + 4u * B > 32u;

  uint32_t gcur = 0xFFFFFFFFu;
  uint64_t gend = 0;
  float bs[4], st[4];
  for (uint64_t tb = (uint64_t)blockIdx.x * TT; tb < p.count; tb += (uint64_t)gridDim.x * TT) {
#pragma unroll
    for (int i = 0; i < kDecR; ++i) {
      const uint64_t tk = tb + pp + (uint64_t)i * P;
      if (tk < p.count) {
        if (gcur == 0xFFFFFFFFu || tk >= gend || tk + p.group < gend) {
          gcur = (uint32_t)(tk / p.group);
          gend = ((uint64_t)gcur + 1u) * p.group;
          const uint16_t* rg = p.ranges_in + (uint64_t)gcur * 2u * dim + 4u * col;
          const u32x2 l = *(const u32x2*)rg, h = *(const u32x2*)(rg + dim);
          const uint16_t l16[4] = {(uint16_t)l.x, (uint16_t)(l.x >> 16), (uint16_t)l.y, (uint16_t)(l.y >> 16)};
          const uint16_t h16[4] = {(uint16_t)h.x, (uint16_t)(h.x >> 16), (uint16_t)h.y, (uint16_t)(h.y >> 16)};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bs[r] = h2f(l16[r]);
            st[r] = kivi_step(bs[r], h2f(h16[r]), levels);
          }
        }
        const uint32_t* cw = p.codes_in + tk * p.nwords;
        const uint32_t lo = cw[wi];
        const uint32_t hi = straddle ? cw[wi + 1] : 0u;
        const uint32_t bits = __builtin_amdgcn_alignbit(hi, lo, sh);
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (float)((bits >> (B * r)) & kMask) * st[r] + bs[r];
        // a token row is written by consecutive lanes as whole cache lines: stream it past the caches
        store_elems<IO, 4>(p.out, tk * dim + 4u * col, o, true);
      }
    }
  }
}

// Group size a multiple of 64: one wave per (group, slab of SW channels), four independent waves per
// workgroup. A lane loads the fp16 ranges of its CPL channels once, then for each 64-token chunk of the
// group issues all its code-word loads before decoding; lane (r, c) holds channels CPL c .. CPL c + CPL - 1 of
// tokens r, r + 64 / TPL, ..., so one store instruction writes 64 CPL / SW whole slab rows. CPL = 8 (16-bit
// output, B <= 4, a dimension of whole slabs only: every lane's eight channels exist) stores 16 bytes per lane
// from one code word, as the float32 path's CPL = 4 does.
template <int B, int SW, int IO, int CPL = 4>
__global__ __launch_bounds__(kBlock) void chan_decode_w(ChanArgs p) {
  static_assert(CPL == 4 || (CPL == 8 && IO != 0 && B <= 4), "eight channels per lane: 16-bit output, one code word");
  constexpr int QW = SW / CPL;      // lanes per slab row
  constexpr int RPI = 64 / QW;      // rows per store instruction
  constexpr int TPL = 64 / RPI;     // tokens per lane per 64-token chunk
  constexpr uint32_t kMask = (1u << B) - 1u;
  const float levels = (float)((1 << B) - 1);
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane / QW, c = lane % QW;
  const uint32_t dim = p.dim, G = p.group;
  const uint32_t slabs = (dim + SW - 1) / SW;
  const uint32_t groups = group_count(p.count, G);
  const uint64_t items = (uint64_t)groups * slabs;
  const uint64_t waves = (uint64_t)gridDim.x * (kBlock / 64);

  for (uint64_t it = (uint64_t)blockIdx.x * (kBlock / 64) + wid; it < items; it += waves) {
    const uint32_t g = (uint32_t)(it / slabs), sl = (uint32_t)(it - (uint64_t)g * slabs);
    const uint32_t first = g * G, n = min(G, p.count - first);
    const uint32_t ch0 = sl * SW, cw = min((uint32_t)SW, dim - ch0);
    const bool cact = (uint32_t)CPL * c < cw;
    const uint32_t ch = ch0 + (cact ? (uint32_t)CPL * c : 0u);
    const uint16_t* rg = p.ranges_in + (uint64_t)g * 2u * dim + ch;
    float bs[CPL], st[CPL];
#pragma unroll
    for (int q = 0; q < CPL / 4; ++q) {
      const u32x2 lw = *(const u32x2*)(rg + 4 * q), hw = *(const u32x2*)(rg + dim + 4 * q);
      const uint16_t l16[4] = {(uint16_t)lw.x, (uint16_t)(lw.x >> 16), (uint16_t)lw.y, (uint16_t)(lw.y >> 16)};
      const uint16_t h16[4] = {(uint16_t)hw.x, (uint16_t)(hw.x >> 16), (uint16_t)hw.y, (uint16_t)(hw.y >> 16)};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        bs[4 * q + k] = h2f(l16[k]);
        st[4 * q + k] = kivi_step(bs[4 * q + k], h2f(h16[k]), levels);
      }
    }
    const uint32_t pos = ch * B, wi = pos >> 5, sh = pos & 31u;
    const bool straddle = sh + (uint32_t)CPL * B > 32u;
    for (uint32_t t0 = 0; t0 < n; t0 += 64) {
      // float32 output, a full 64-token chunk of a full slab: every lane is active and no row is clamped, so each
      // load and store is a wave-uniform row base plus the lane's 32-bit byte offset (config-3 decode +5 %; with
      // 16-bit output the same path measured 5-7 % slower, so those keep the general path)
      if (IO == 0 && n - t0 >= 64u && cw == (uint32_t)SW) {
        constexpr uint32_t ES = 4u;  // bytes per output element
        const char* cb = (const char*)(p.codes_in + (uint64_t)(first + t0) * p.nwords);
        char* ob = (char*)p.out + ((uint64_t)(first + t0) * dim) * ES;
        const uint32_t cl = (r * p.nwords + wi) * 4u, ol = (r * dim + ch) * ES;
        uint32_t lo[TPL], hi[TPL];
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
          const uint32_t* w = (const uint32_t*)(cb + (uint64_t)(RPI * i) * p.nwords * 4u + cl);
          lo[i] = w[0];
          hi[i] = straddle ? w[1] : 0u;
        }
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
          const uint32_t bits = __builtin_amdgcn_alignbit(hi[i], lo[i], sh);
          float o[CPL];
#pragma unroll
          for (int k = 0; k < CPL; ++k) o[k] = (float)((bits >> (B * k)) & kMask) * st[k] + bs[k];
          store_elems<IO, CPL>(ob + (uint64_t)(RPI * i) * dim * ES + ol, 0, o, PITCH_KIVI_DEC_NTS);
        }
        continue;
      }
      const uint32_t* cwp = p.codes_in + (uint64_t)(first + t0) * p.nwords + wi;
      uint32_t lo[TPL], hi[TPL];
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        const uint32_t tk = t0 + r + RPI * i;
        const uint32_t tc = (tk < n ? tk : n - 1) - t0;  // rows past the group's end re-read its last row
        lo[i] = cwp[(uint64_t)tc * p.nwords];
        hi[i] = straddle ? cwp[(uint64_t)tc * p.nwords + 1] : 0u;
      }
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        const uint32_t tk = t0 + r + RPI * i;
        if (tk < n && cact) {
          const uint32_t bits = __builtin_amdgcn_alignbit(hi[i], lo[i], sh);
          float o[CPL];
#pragma unroll
          for (int k = 0; k < CPL; ++k) o[k] = (float)((bits >> (B * k)) & kMask) * st[k] + bs[k];
          store_elems<IO, CPL>(p.out, (uint64_t)(first + tk) * dim + ch, o, PITCH_KIVI_DEC_NTS);
        }
      }
    }
  }
}

template <int B, int IO>
__global__ __launch_bounds__(kBlock) void chan_decode1(ChanArgs p) {
  const float levels = (float)((1 << B) - 1);
  constexpr uint32_t kMask = (1u << B) - 1u;
  const uint64_t total = (uint64_t)p.count * p.dim;
  for (uint64_t idx = (uint64_t)blockIdx.x * kBlock + threadIdx.x; idx < total;
       idx += (uint64_t)gridDim.x * kBlock) {
    const uint64_t tok = idx / p.dim;
    const uint32_t ch = (uint32_t)(idx - tok * p.dim);
    const uint64_t g = tok / p.group;
    const float base = h2f(p.ranges_in[g * 2u * p.dim + ch]);
    const float step = kivi_step(base, h2f(p.ranges_in[g * 2u * p.dim + p.dim + ch]), levels);
    const uint32_t* cw = p.codes_in + tok * p.nwords;
    const uint32_t pos = ch * B, wi = pos >> 5, sh = pos & 31u;
    const uint32_t lo = cw[wi], hi = (sh + B > 32u) ? cw[wi + 1] : 0u;
    const uint32_t code = __builtin_amdgcn_alignbit(hi, lo, sh) & kMask;
    const float o[1] = {(float)code * step + base};
    store_elems<IO, 1>(p.out, idx, o, false);
  }
}

template <int B, int IO>
hipError_t launch_b(bool encode, const ChanArgs& a, hipStream_t s) {
  const bool vec4 = (a.dim & 3u) == 0u;
  if (encode && vec4 && a.group <= (uint32_t)kGroupMaxW) {
    const uint64_t groups = ((uint64_t)a.count + a.group - 1) / a.group;
    // 32-channel slabs double the work items and halve each lane's registers, which balances float32 calls
    // with few (group, 64-channel) items over the resident waves (+5-10 % at 4096-8192 items); long calls keep
    // 64-channel slabs, whose loads read whole 256-byte rows (+4 % at 131072 items). With 16-bit keys a
    // 64-channel row is only 128 bytes and the wider slab measured 6-7 % faster at 4096 items as well.
    const uint64_t items64 = groups * ((a.dim + 63) / 64);
    const int sw = PITCH_KIVI_SLAB ? PITCH_KIVI_SLAB : (IO == 0 && items64 <= 32768 ? 32 : 64);
    const bool dp = PITCH_KIVI_DP && (B == 2 || B == 4 || B == 8) && a.dim % (uint32_t)sw == 0u;  // full slabs
    auto go = [&](auto sw_c, auto dp_c) {
      constexpr int SW = decltype(sw_c)::value;
      constexpr bool DP = decltype(dp_c)::value;
      const uint64_t items = groups * ((a.dim + SW - 1) / SW);
      const void* k = (const void*)&chan_encode_w<B, IO, SW, DP>;
      // float32 keys: balanced rounds (config 3 is 1.33 rounds at full occupancy); the 16-bit encoders are
      // bound by their arithmetic and keep every resident wave
      const uint64_t grid = persistent_grid(k, (items + 3) / 4, kBlock, PITCH_KIVI_BALANCE && IO == 0);
      const uint64_t need = (items + 3) / 4;
      const uint64_t min_rounds = SW == 32 ? PITCH_KIVI_ENC_MIN_ROUNDS32 : PITCH_KIVI_ENC_MIN_ROUNDS;
      const int cap = SW == 32 ? PITCH_KIVI_ENC_WG_PER_CU32 : PITCH_KIVI_ENC_WG_PER_CU;
      if (PITCH_KIVI_ENC_ONE_LAUNCH && IO == 0 && need >= min_rounds * grid) {
        // float32 calls of min_rounds+ rounds: one launch of one item per wave, far more workgroups than the CUs
        // hold (config-5 keys, 341 rounds: 5.52 TB/s against 5.41 for launches of two rounds, three repeats each,
        // before the cap), held at cap workgroups per CU (0: the kernel's full residency)
        const uint64_t g = need < 0x7FFFFFFFull ? need : 0x7FFFFFFFull;
        hipLaunchKernelGGL((chan_encode_w<B, IO, SW, DP>), dim3((uint32_t)g), dim3(kBlock),
                           lds_cap_bytes(k, cap), s, a);
        return;
      }
      const uint64_t slabs = (a.dim + SW - 1) / SW, rounds = slice_rounds(kChanSliceRoundsEnc);
      if (rounds && (items + 3) / 4 > grid * rounds && grid * rounds * 4 >= slabs) {
        const uint64_t gpl = grid * rounds * 4 / slabs;  // groups per launch
        constexpr uint64_t ES = IO == 0 ? 4 : 2;
        for (uint64_t g0 = 0; g0 < groups; g0 += gpl) {
          const uint64_t t0 = g0 * a.group;
          ChanArgs b = a;
          b.count = (uint32_t)((uint64_t)a.count - t0 < gpl * a.group ? (uint64_t)a.count - t0 : gpl * a.group);
          b.in = (const char*)a.in + t0 * a.dim * ES;
          b.codes_out = a.codes_out + t0 * a.nwords;
          b.ranges_out = a.ranges_out + g0 * 2 * a.dim;
          const uint64_t gb = ((uint64_t)b.count + a.group - 1) / a.group, nb = (gb * slabs + 3) / 4;
          hipLaunchKernelGGL((chan_encode_w<B, IO, SW, DP>), dim3((uint32_t)(nb < grid ? nb : grid)), dim3(kBlock), 0,
                             s, b);
        }
        return;
      }
      hipLaunchKernelGGL((chan_encode_w<B, IO, SW, DP>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
    };
    using I32 = std::integral_constant<int, 32>;
    using I64 = std::integral_constant<int, 64>;
    constexpr bool kDP = B == 2 || B == 4 || B == 8;
    if (sw == 32) {
      if (dp) go(I32{}, std::integral_constant<bool, kDP>{});
      else go(I32{}, std::false_type{});
    } else {
      if (dp) go(I64{}, std::integral_constant<bool, kDP>{});
      else go(I64{}, std::false_type{});
    }
  } else if (encode) {
    const uint64_t groups = ((uint64_t)a.count + a.group - 1) / a.group;
    const void* k = vec4 ? (const void*)&chan_encode4<B, IO> : (const void*)&chan_encode1<B, IO>;
    const uint64_t grid = persistent_grid(k, groups);
    if (vec4) hipLaunchKernelGGL((chan_encode4<B, IO>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
    else hipLaunchKernelGGL((chan_encode1<B, IO>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  } else if (vec4 && a.group % 64u == 0u) {
    // float32 output: 32-channel slabs for calls with few (group, 64-channel) items, which then fill the
    // resident waves (config-3 decode +3-4 % back-to-back, within 0.5 % in kernel time); 16-bit output keeps
    // 64-channel slabs (a 32-channel slab's rows are 64 bytes: 22 % slower)
    const uint64_t groups = ((uint64_t)a.count + a.group - 1) / a.group;
    const uint64_t items64 = groups * ((a.dim + kSlab - 1) / kSlab);
    auto go = [&](auto sw_c, auto cpl_c) {
      constexpr int SW = decltype(sw_c)::value, CPL = decltype(cpl_c)::value;
      const uint64_t items = groups * ((a.dim + SW - 1) / SW);
      const uint64_t grid = persistent_grid((const void*)&chan_decode_w<B, SW, IO, CPL>, (items + 3) / 4);
      if (IO == 0 && PITCH_KIVI_DEC_ONE_LAUNCH && (items + 3) / 4 >= PITCH_KIVI_DEC_MIN_ROUNDS * grid) {
        // one launch of one item per wave at a capped residency (above); the kernel's grid-stride loop covers
        // any items past 2^31 - 1 workgroups
        const uint64_t need = (items + 3) / 4, g = need < 0x7FFFFFFFull ? need : 0x7FFFFFFFull;
        const void* k = (const void*)&chan_decode_w<B, SW, IO, CPL>;
        hipLaunchKernelGGL((chan_decode_w<B, SW, IO, CPL>), dim3((uint32_t)g), dim3(kBlock),
                           lds_cap_bytes(k, PITCH_KIVI_DEC_WG_PER_CU), s, a);
        return;
      }
      const uint64_t slabs = (a.dim + SW - 1) / SW, rounds = slice_rounds(kChanSliceRoundsDec);
      if (rounds && (items + 3) / 4 > grid * rounds && grid * rounds * 4 >= slabs) {
        const uint64_t gpl = grid * rounds * 4 / slabs;  // groups per launch
        constexpr uint64_t ES = IO == 0 ? 4 : 2;
        for (uint64_t g0 = 0; g0 < groups; g0 += gpl) {
          const uint64_t t0 = g0 * a.group;
          ChanArgs b = a;
          b.count = (uint32_t)((uint64_t)a.count - t0 < gpl * a.group ? (uint64_t)a.count - t0 : gpl * a.group);
          b.codes_in = a.codes_in + t0 * a.nwords;
          b.ranges_in = a.ranges_in + g0 * 2 * a.dim;
          b.out = (char*)a.out + t0 * a.dim * ES;
          const uint64_t gb = ((uint64_t)b.count + a.group - 1) / a.group, nb = (gb * slabs + 3) / 4;
          hipLaunchKernelGGL((chan_decode_w<B, SW, IO, CPL>), dim3((uint32_t)(nb < grid ? nb : grid)), dim3(kBlock), 0, s, b);
        }
        return;
      }
      hipLaunchKernelGGL((chan_decode_w<B, SW, IO, CPL>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
    };
    // 16-bit output at B <= 4 with whole slabs, long calls: eight channels per lane (16-byte stores from one code
    // word); same output bits as four
    constexpr int kCpl16 = IO != 0 && B <= 4 && PITCH_KIVI_DEC_CPL8 ? 8 : 4;
    using Cpl4 = std::integral_constant<int, 4>;
    if (PITCH_KIVI_DEC_SLAB32 && IO == 0 && items64 <= PITCH_KIVI_DEC_SLAB32_MAX)
      go(std::integral_constant<int, 32>{}, Cpl4{});
    else if (kCpl16 == 8 && a.dim % kSlab == 0u && items64 >= PITCH_KIVI_DEC_CPL8_MIN_ITEMS)
      go(std::integral_constant<int, kSlab>{}, std::integral_constant<int, kCpl16>{});
    else go(std::integral_constant<int, kSlab>{}, Cpl4{});
  } else if (vec4) {
    const uint32_t P = kBlock / (a.dim >> 2);
    const uint64_t need = ((uint64_t)a.count + P * kDecR - 1) / (P * kDecR);
    const uint64_t grid = persistent_grid((const void*)&chan_decode4<B, IO>, need);
    hipLaunchKernelGGL((chan_decode4<B, IO>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  } else {
    const uint64_t need = ((uint64_t)a.count * a.dim + kBlock - 1) / kBlock;
    const uint64_t grid = persistent_grid((const void*)&chan_decode1<B, IO>, need);
    hipLaunchKernelGGL((chan_decode1<B, IO>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

#if PITCH_IO == 0
// ------------------------------------------------------------------------------------------- pack
__global__ __launch_bounds__(kBlock) void pack_generic(PackArgs p) {
  const uint32_t nwords = (p.dim * p.bits + 31u) / 32u;
  const uint64_t total = p.count * nwords;
  for (uint64_t w = (uint64_t)blockIdx.x * kBlock + threadIdx.x; w < total; w += (uint64_t)gridDim.x * kBlock) {
    const uint64_t row = w / nwords;
    const uint32_t wi = (uint32_t)(w - row * nwords);
    const uint8_t* src = p.unpacked_in + row * p.dim;
    const uint32_t mask = (1u << p.bits) - 1u;
    uint32_t word = 0u;
    for (uint32_t i = (32u * wi) / p.bits; i < p.dim; ++i) {
      const int s = (int)(i * p.bits) - (int)(32u * wi);
      if (s >= 32) break;
      const uint32_t c = src[i] & mask;
      word |= s >= 0 ? (c << s) : (c >> (-s));
    }
    p.packed_out[w] = word;
  }
}

__global__ __launch_bounds__(kBlock) void unpack_generic(PackArgs p) {
  const uint32_t nwords = (p.dim * p.bits + 31u) / 32u;
  const uint64_t total = p.count * p.dim;
  const uint32_t mask = (1u << p.bits) - 1u;
  for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (uint64_t)gridDim.x * kBlock) {
    const uint64_t row = i / p.dim;
    const uint32_t c = (uint32_t)(i - row * p.dim);
    const uint32_t* w = p.packed_in + row * nwords;
    const uint32_t pos = c * p.bits, wi = pos >> 5, sh = pos & 31u;
    const uint32_t lo = w[wi], hi = (sh + p.bits > 32u) ? w[wi + 1] : 0u;
    p.unpacked_out[i] = (uint8_t)(__builtin_amdgcn_alignbit(hi, lo, sh) & mask);
  }
}

#endif  // PITCH_IO == 0

}  // namespace

#define PITCH_CAT2(a, b) a##b
#define PITCH_CAT(a, b) PITCH_CAT2(a, b)

hipError_t PITCH_CAT(launch_channel_io, PITCH_IO)(bool encode, int bits, const ChanArgs& a, hipStream_t s) {
  switch (bits) {
    case 2: return launch_b<2, PITCH_IO>(encode, a, s);
    case 3: return launch_b<3, PITCH_IO>(encode, a, s);
    case 4: return launch_b<4, PITCH_IO>(encode, a, s);
    case 5: return launch_b<5, PITCH_IO>(encode, a, s);
    case 6: return launch_b<6, PITCH_IO>(encode, a, s);
    case 7: return launch_b<7, PITCH_IO>(encode, a, s);
    case 8: return launch_b<8, PITCH_IO>(encode, a, s);
    default: return hipErrorInvalidValue;
  }
}

#if PITCH_IO == 0
hipError_t launch_pack(bool pack, const PackArgs& a, hipStream_t s) {
  if (pack) {
    const uint64_t nwords = (a.dim * a.bits + 31u) / 32u;
    const uint64_t grid = persistent_grid((const void*)&pack_generic, (a.count * nwords + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(pack_generic, dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  } else {
    const uint64_t grid =
        persistent_grid((const void*)&unpack_generic, (a.count * a.dim + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(unpack_generic, dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

// Self-test of rcp_rn: thread t checks the positive normal floats with bit patterns first + t * per + k
// (k < per, below 2^126), counting those whose rcp_rn differs from the correctly rounded 1 / x (the library is
// built with -fhip-fp32-correctly-rounded-divide-sqrt). One count per thread, no atomics.
__global__ __launch_bounds__(kBlock) void selftest_reciprocal(uint32_t* counts, uint32_t first, uint32_t end,
                                                                 uint32_t per) {
  const uint32_t t = blockIdx.x * kBlock + threadIdx.x;
  uint32_t bad = 0;
  for (uint32_t k = 0; k < per; ++k) {
    const uint64_t bits = (uint64_t)first + (uint64_t)t * per + k;
    if (bits >= end) break;
    const float x = __uint_as_float((uint32_t)bits);
    bad += __float_as_uint(rcp_rn(x)) != __float_as_uint(1.0f / x) ? 1u : 0u;
  }
  counts[t] = bad;
}

hipError_t launch_selftest_reciprocal(uint32_t* counts, uint32_t threads, uint32_t first, uint32_t end,
                                      hipStream_t s) {
  if (threads % kBlock != 0 || end <= first) return hipErrorInvalidValue;
  const uint32_t per = (uint32_t)(((uint64_t)end - first + threads - 1) / threads);
  hipLaunchKernelGGL(selftest_reciprocal, dim3(threads / kBlock), dim3(kBlock), 0, s, counts, first, end, per);
  return hipGetLastError();
}
#endif

}  // namespace pitch
