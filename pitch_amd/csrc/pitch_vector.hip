// Per-vector TurboQuant and single-level PolarQuant encode/decode for one dimension (PITCH_DIM) and one
// element type of the uncompressed vectors (PITCH_IO: 0 float32, 1 float16, 2 bfloat16).
//
// Encode follows reference/pitch_reference.py:92-102 (TurboQuant) and :109-121 (PolarQuant); decode
// :104-107 and :123-129. The Metal kernels they replace are PITCHKernels.metal:114-246, which run one
// threadgroup per vector with one coordinate per thread and two barriers per transform stage; here a
// vector lives in the registers of a small team of lanes, transform stages run in registers or through
// DPP lane exchanges, and one workgroup processes 64 vectors per iteration of a grid-stride loop.
//
// Numerics. The encoders rotate in float64 with exact butterflies in the reference's stage order, so the
// rotated coordinates agree with the float64 specification to a few ulps (PolarQuant: bit for bit, with
// correctly rounded divisions) and codes can differ only for values within ~1e-15 of a decision edge. The
// decoders run in float32 (relative L2 error ~1e-7 against the float64 specification).
#include <cstddef>

#include "pitch_device.h"

#ifndef PITCH_DIM
#error "compile with -DPITCH_DIM=<dim>"
#endif
#ifndef PITCH_IO
#define PITCH_IO 0
#endif
#ifndef PITCH_LPV_EMAX
#define PITCH_LPV_EMAX 32  // most coordinates one lane of the TurboQuant encoder holds
#endif
#ifndef PITCH_QBATCH
#define PITCH_QBATCH 15  // bucket-table lookups issued before the first is used (the LDS counter tracks 15)
#endif
#ifndef PITCH_ENC_PREFETCH
#define PITCH_ENC_PREFETCH 1  // 1: the TurboQuant encoder loads block i+1 while it computes block i
#endif
#ifndef PITCH_ENC_WAVES
#define PITCH_ENC_WAVES 2  // waves per SIMD the TurboQuant encoder's register budget must allow
#endif

namespace pitch {
namespace {

template <int D>
struct DimConst {
  static constexpr bool kPow4 = (ilog2(D) % 2) == 0;
  // math.sqrt(D) in float64: exact for powers of 4, else 2^k * RN(sqrt(2)).
  static constexpr double kSqrt =
      kPow4 ? double(1 << (ilog2(D) / 2)) : 0x1.6a09e667f3bcdp+0 * double(1 << (ilog2(D) / 2));
  static constexpr double kInvSqrt = 1.0 / kSqrt;
  static constexpr float kInvSqrtF = float(kInvSqrt);
};

// One segment of an encode: count vectors from in to codes_out / scales_out. A single call has one (the call's
// own buffers); a batched launch gives each of its workgroups the segment that block_start assigns it.
struct EncSeg {
  const void* in;
  uint32_t* codes_out;
  float* scales_out;
  uint64_t count;
};
__device__ __forceinline__ EncSeg call_segment(const VecArgs& p) {
  return EncSeg{p.in, p.codes_out, p.scales_out, p.count};
}
// The segment of this workgroup in a batched launch, and the workgroup's index and count within it.
struct BatchSlot {
  EncSeg seg;
  uint64_t block, blocks;
};
// The segment of workgroup blockIdx.x: the number of segments after the first that start at or before it (block_start
// is non-decreasing). Uniform (kernel arguments and the block index); unrolled, so the scalar loads of block_start go
// out together instead of one dependent load per segment.
template <typename Args>
__device__ __forceinline__ uint32_t batch_item(const Args& pb) {
  uint32_t i = 0;
#pragma unroll
  for (uint32_t j = 1; j < kBatchItems; ++j) i += (j < pb.items && pb.block_start[j] <= blockIdx.x) ? 1u : 0u;
  return i;
}
__device__ __forceinline__ BatchSlot batch_slot(const VecBatchArgs& pb) {
  const uint32_t i = batch_item(pb);
  return BatchSlot{EncSeg{pb.in[i], pb.codes_out[i], pb.scales_out[i], pb.count[i]},
                   (uint64_t)(blockIdx.x - pb.block_start[i]), (uint64_t)(pb.block_start[i + 1] - pb.block_start[i])};
}

constexpr double kTwoPi = 0x1.921fb54442d18p+2;  // 2 * np.pi

// Fast PolarQuant quantisation. A radius or angle code is floor(t) with t = value * levels + 0.5
// (pitch_reference.py:116-117). The encoder first evaluates t in float32; when t is at least kPolarGuard
// from an integer, floor(t) is certain and used. Otherwise (and for a pair at the origin) the float64 path
// that follows the reference's operation order decides. kPolarGuard is about four times the worst float32
// error of t at b = 8 (radius: under 7e-5; angle: under 1e-4), so only pairs within 3e-4 of a rounding
// point take the float64 path.
constexpr float kPolarGuard = 3e-4f;

// theta / (2 pi) in [0, 1] of the direction (a, c) = atan2(c, a) mod 2 pi, in float32: octant reduction and
// atan(z) = z * P(z^2) on [0, 1] with the least-squares polynomial gen_tables.py fits for bit width B, whose
// error keeps t = turns * 2^B + 0.5 within 1e-4 of its exact value.
template <int B>
__device__ __forceinline__ float angle_turns(float c, float a) {
  constexpr int DEG = pitch_atan_degree(B);
  const float ax = __builtin_fabsf(a), ay = __builtin_fabsf(c);
  const float mx = __builtin_fmaxf(ax, ay), mn = __builtin_fminf(ax, ay);
  const float z = mn * __builtin_amdgcn_rcpf(mx);
  const float s = z * z;
  float poly = pitch_atan_coef[DEG][DEG];
#pragma unroll
  for (int i = DEG - 1; i >= 0; --i) poly = __builtin_fmaf(poly, s, pitch_atan_coef[DEG][i]);
  float at = poly * z;                                   // atan(mn / mx) in [0, pi / 4]
  if (ay > ax) at = 0x1.921fb6p+0f - at;                 // pi / 2 - at
  if (a < 0.f) at = 0x1.921fb6p+1f - at;                 // pi - at
  const float turns = at * 0x1.45f306p-3f;               // / (2 pi), in [0, 0.5]
  return c < 0.f ? 1.f - turns : turns;
}

// Radius and angle codes of the pair (a, c) with r2 = a^2 + c^2 in float64, in the reference's order
// (pitch_reference.py:111-117): floor(r / rmax * (2^B - 1) + 0.5) clipped, floor(theta / 2 pi * 2^B + 0.5)
// mod 2^B with theta = atan2(c, a) mod 2 pi. Out of line: only pairs near a rounding point come here.
template <int B>
__device__ __attribute__((noinline)) uint2 polar_codes_exact(double a, double c, double r2, double safe) {
  constexpr int L = 1 << B;
  constexpr double RL = double(L - 1), N = double(L);
  double rq = __builtin_floor(__builtin_sqrt(r2) / safe * RL + 0.5);
  rq = rq < 0.0 ? 0.0 : (rq > RL ? RL : rq);
  double th = atan2(c, a);
  if (th < 0.0) th += kTwoPi;  // np.mod(theta, 2 pi) for theta in [-pi, 0)
  const double tq = __builtin_floor(th / kTwoPi * N + 0.5);
  return make_uint2((uint32_t)rq, (uint32_t)tq & (uint32_t)(L - 1));
}

// floor(t) when t is at least kPolarGuard from an integer (then ok is left alone), else ok = false.
__device__ __forceinline__ float guarded_floor(float t, bool& ok) {
  const float k = __builtin_floorf(t);
  const float f = t - k;
  ok = ok && f > kPolarGuard && f < 1.f - kPolarGuard;
  return k;
}

// The staged-stage PolarQuant encoder's angle in sector units, w = (atan2(c, a) mod 2 pi) * 2^B / (2 pi) in
// [0, 2^B]: angle_turns with the factor 2^B / (2 pi) folded into the polynomial's coefficients (each product
// rounded once to float32) and the octant fix-ups taken in sector units (2^B / 4, 2^B / 2, 2^B are exact).
template <int B>
__device__ __forceinline__ float angle_sectors(float c, float a) {
  constexpr int DEG = pitch_atan_degree(B);
  constexpr float L = float(1 << B);
  constexpr float kS = float(double(1 << B) / 6.283185307179586);  // 2^B / (2 pi)
  const float ax = __builtin_fabsf(a), ay = __builtin_fabsf(c);
  const float mx = __builtin_fmaxf(ax, ay), mn = __builtin_fminf(ax, ay);
  const float z = mn * __builtin_amdgcn_rcpf(mx);
  const float s = z * z;
  float poly = pitch_atan_coef[DEG][DEG] * kS;
#pragma unroll
  for (int i = DEG - 1; i >= 0; --i) poly = __builtin_fmaf(poly, s, pitch_atan_coef[DEG][i] * kS);
  float w = poly * z;                  // atan(mn / mx) in sector units, [0, 2^B / 8]
  if (ay > ax) w = 0.25f * L - w;
  if (a < 0.f) w = 0.5f * L - w;
  return c < 0.f ? L - w : w;
}

// floor(t) for t >= 0 (a truncating convert) when t is at least kPolarGuard from an integer (then ok is left
// alone), else ok = false; a NaN t fails the guard.
__device__ __forceinline__ uint32_t guarded_code(float t, bool& ok) {
  const float f = __builtin_amdgcn_fractf(t);
  ok = ok && f > kPolarGuard && f < 1.f - kPolarGuard;
  return (uint32_t)t;
}

// floor(u + g) for u + g >= 0 from u = t - g, when t lies at least g from an integer: then fract(u) < 1 - 2g
// and floor(u) = floor(t) (ok is left alone); else ok = false. A NaN u fails.
__device__ __forceinline__ uint32_t guarded_code_shifted(float u, float g, bool& ok) {
  ok = ok && __builtin_amdgcn_fractf(u) < 1.f - 2.f * g;
  return (uint32_t)u;
}

// Guard of the staged-stage encoder's radius t = sqrt_f32(fma(a, a, RN(c c))) * RN((2^B - 1) / rmax) + 0.5 on the
// float32 pair (a, c), whose error is under (2^B - 1) * 4e-7 (the pair's roundings, two in the squared radius,
// a square root within an ulp, the scale's rounding and the fused add): (2^B - 1) * 1.2e-6, three times that.
template <int B>
constexpr float polar_radius_guard() { return float((1 << B) - 1) * 1.2e-6f; }

// Angle codes at B <= 5 by comparisons with the sector boundaries instead of an arctangent. Code k of
// floor(theta / (2 pi) * 2^B + 0.5) mod 2^B (pitch_reference.py:117) covers the directions from (k - 1/2) to
// (k + 1/2) sectors. In the first octant, with mx = max(|a|, |c|) and mn = min(|a|, |c|), the direction's
// angle atan(mn / mx) lies past boundary j (angle (j - 1/2) 2 pi / 2^B, j = 1 .. ceil(2^B / 8)) exactly when
// d_j = mn - mx tan_j > 0. d_j = fma(mx, -RN(tan_j), mn) errs by under 2.4e-7 mx (the roundings of mn, mx and
// tan_j to float32, and of the fused result) for mx >= 1e-30 (products far from float32's subnormals), so a
// decision with |d_j| > 2e-6 mx is certain; otherwise, or for mx < 1e-30 (the origin included), the float64
// path decides. The octant's reflections map the first-octant code n1 to L/4 - n1 (|c| > |a|), L/2 - n
// (a negative) and L - n (c negative), exact on integers: a first-octant direction at a boundary fails the
// guard, and for B >= 3 the octant edges are sector centres; at B = 2 the edge pi / 4 is the one boundary
// (tan = 1). A zero of either sign on an axis reflects onto itself, so the sign bit alone is tested.
template <int B>
constexpr int polar_sector_bounds() { return ((1 << B) + 7) / 8; }
constexpr float kSectorGuard = 2e-6f;

template <int B>
__device__ __forceinline__ uint32_t sector_code(float c, float a, bool& ok) {
  constexpr int L = 1 << B, K = polar_sector_bounds<B>();
  static_assert(B >= 2 && B <= 5 && K <= 4, "sector boundaries of the first octant");
  const float ax = __builtin_fabsf(a), ay = __builtin_fabsf(c);
  const float mx = __builtin_fmaxf(ax, ay), mn = __builtin_fminf(ax, ay);
  const float gm = kSectorGuard * mx;
  bool good = mx >= 1e-30f;
  uint32_t n = 0;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float dj = __builtin_fmaf(mx, -pitch_sector_tan[B - 2][j], mn);
    n += dj > 0.f ? 1u : 0u;
    good = good && __builtin_fabsf(dj) > gm;
  }
  ok = ok && good;
  n = ay > ax ? (uint32_t)(L / 4) - n : n;
  n = __float_as_uint(a) >> 31 ? (uint32_t)(L / 2) - n : n;
  n = __float_as_uint(c) >> 31 ? (uint32_t)L - n : n;
  return n & (uint32_t)(L - 1);
}

// sector_code as one LDS byte lookup indexed by sign bits: bit 0 the sign of c, bit 1 the sign of a, bit 2 the
// sign of |a| - |c| (set exactly when |c| > |a|: the difference of distinct floats is nonzero, of equal ones +0),
// bits 3 .. K + 2 the signs of d_{K-1} .. d_0. Each bit is appended with one v_alignbit(idx, x, 31) =
// (idx << 1) | (x >> 31). The table holds, for every index, the code the octant reflections give to the
// first-octant count n = the number of clear d_j sign bits. An accepted pair has every |d_j| above the guard,
// so no d_j is zero and a clear sign bit means d_j > 0. The guard is gm = fma(mx, 2e-6, 1e-36): for mx < 1e-36
// it exceeds mx >= |d_j| and rejects the pair (the origin included); above, the products mx tan_j (tan_j >=
// 0.098) are normal floats and d_j errs by under 2.4e-7 mx + 2^-149 (2^-150 for each subnormal rounding of mn
// and of the fused result), a third of gm at most. The staged encoders take the float32 path only for vectors
// whose largest radius is at least 1e-15, where a pair below 1e-30 has radius code 0 however its square rounds.
// The 16 - 128 byte table sits in at most 32 banks, so a wave's lookups never conflict (lanes reading one dword
// are served by a broadcast).
#ifndef PITCH_POLAR_OCT_TAB
#define PITCH_POLAR_OCT_TAB 1  // PolarQuant's staged and transposed encoders take their angle codes from the table
#endif
template <int B>
struct OctTab {
  static constexpr int K = polar_sector_bounds<B>();
  static constexpr int N = K <= 4 ? 1 << (K + 3) : 1;  // b > 5 takes no table
};
typedef __attribute__((address_space(3))) const uint8_t lds_u8_t;

template <int B>
__device__ __forceinline__ void octant_table_build(uint8_t* tab, int tid, int nthreads) {
  using O = OctTab<B>;
  constexpr uint32_t L = 1u << B;
  for (int i = tid; i < O::N; i += nthreads) {
    uint32_t n = 0;
#pragma unroll
    for (int j = 0; j < O::K; ++j) n += ((i >> (3 + j)) & 1) ? 0u : 1u;
    n = ((i >> 2) & 1) ? L / 4 - n : n;
    n = ((i >> 1) & 1) ? L / 2 - n : n;
    n = (i & 1) ? L - n : n;
    tab[i] = (uint8_t)(n & (L - 1));
  }
}

template <int B>
__device__ __forceinline__ uint32_t sector_code_tab(float c, float a, bool& ok, lds_u8_t* tab) {
  using O = OctTab<B>;
  static_assert(B >= 2 && B <= 5 && O::K <= 4, "sector boundaries of the first octant");
  const float ax = __builtin_fabsf(a), ay = __builtin_fabsf(c);
  const float mx = __builtin_fmaxf(ax, ay), mn = __builtin_fminf(ax, ay);
  const float gm = __builtin_fmaf(mx, kSectorGuard, 1e-36f);
  bool good = true;
  uint32_t idx = 0;
#pragma unroll
  for (int j = 0; j < O::K; ++j) {
    const float dj = __builtin_fmaf(mx, -pitch_sector_tan[B - 2][j], mn);
    idx = j == 0 ? __float_as_uint(dj) >> 31 : __builtin_amdgcn_alignbit(idx, __float_as_uint(dj), 31);
    good = good && __builtin_fabsf(dj) > gm;
  }
  ok = ok && good;
  idx = __builtin_amdgcn_alignbit(idx, __float_as_uint(ax - ay), 31);
  idx = __builtin_amdgcn_alignbit(idx, __float_as_uint(a), 31);
  idx = __builtin_amdgcn_alignbit(idx, __float_as_uint(c), 31);
  return tab[idx];
}

// y / sqrt(D) rounded as the reference's division (pitch_reference.py:33).
template <int D>
__device__ __forceinline__ double div_sqrt_d(double y) {
  using C = DimConst<D>;
  if constexpr (C::kPow4) return y * C::kInvSqrt;
  else return y / C::kSqrt;
}

// Key-bias offset of coordinates [c, c + N) of vector v: o = b_h * cos_t + rotate_half(b_h) * sin_t with
// rotate_half(x) = (-x[D/2:], x[:D/2]) (reference/mechanism_eval.py:88-97), each product and the sum rounded once
// as the reference's float32 torch expression rounds them (the library is built with -ffp-contract=off).
template <int D, int N>
__device__ __forceinline__ void key_bias_offset(const VecArgs& p, uint64_t v, int c, float (&o)[N]) {
  uint64_t tok;
  uint32_t h;
  if (p.count <= 0xFFFFFFFFull) {  // 32-bit division whenever the call allows it
    const uint32_t v32 = (uint32_t)v, t32 = v32 / p.kb_heads;
    tok = t32;
    h = v32 - t32 * p.kb_heads;
  } else {
    tok = v / p.kb_heads;
    h = (uint32_t)(v - tok * p.kb_heads);
  }
  const float* b = p.kb_bias + (uint64_t)h * D;
  const float* cs = p.kb_cos + (p.kb_first + tok) * D;
  const float* sn = p.kb_sin + (p.kb_first + tok) * D;
  if constexpr (N % 4 == 0 && D >= 8) {
    // four coordinates at a time; a 4-aligned group never straddles the halves
#pragma unroll
    for (int r = 0; r < N; r += 4) {
      const int j = c + r;
      const bool lo = j < D / 2;
      const f32x4 bv = *(const f32x4*)(b + j);
      const f32x4 pv = *(const f32x4*)(b + (lo ? j + D / 2 : j - D / 2));
      const f32x4 cv = *(const f32x4*)(cs + j);
      const f32x4 sv = *(const f32x4*)(sn + j);
      const float bs[4] = {bv.x, bv.y, bv.z, bv.w}, ps[4] = {pv.x, pv.y, pv.z, pv.w};
      const float cc[4] = {cv.x, cv.y, cv.z, cv.w}, ss[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float t1 = bs[k] * cc[k];
        const float t2 = (lo ? -ps[k] : ps[k]) * ss[k];
        o[r + k] = t1 + t2;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < N; ++r) {
      const int j = c + r;
      const float rh = j < D / 2 ? -b[j + D / 2] : b[j - D / 2];
      const float t1 = b[j] * cs[j];
      const float t2 = rh * sn[j];
      o[r] = t1 + t2;
    }
  }
}

// TurboQuant quantiser: code = #{edges < u}, searchsorted(edges, u, 'left') (pitch_reference.py:99-101).
// With a bucket table (gen_tables.py lut_for): bucket j = floor(u * 2^m + off), clamped to [0, n), holds at
// most one edge e_j, and code = c_j + [u > e_j]. The comparison is made in the bucket domain: one fma gives
// t = u * 2^m + off + 2^16 + 2^15 in float64, which lies in [2^16, 2^17) for every |u| <= 1, so the top 20
// mantissa bits (the high word's low 20 bits) are floor(16 * (t - 2^16)) and bits 4 .. 19 of the high word
// hold the bucket index plus 2^15. A med3 clamp of the high word and a mask give the byte offset 16 * j of
// the entry directly. Each entry holds E_j = e_j * 2^m + off + 2^16 + 2^15 (exact in float64: 2^m is a
// power of two) and c_j, and t > E_j decides the code: it equals u > e_j except where u lies within the
// rounding of t (2^-37 bucket units) of the edge, far inside the near-boundary band. Lookups are issued in
// batches of up to 15 (what the LDS wait counter tracks) before any result is used, so a wave pays one LDS
// round trip per batch, not per coordinate. Tables too large for LDS use a binary search over the float64
// edges.
template <int D, int B>
struct TqQuant {
  static constexpr int L = 1 << B;
  static constexpr PitchLutInfo LI = pitch_lut_info(ilog2(D), B);
  static constexpr bool kLut = LI.offset >= 0;
  static constexpr int kBatch = PITCH_QBATCH;
  static constexpr double kMagic = 98304.0 + LI.off;  // 2^16 + 2^15 + off
  static constexpr int kIdxBits = kLut ? ilog2(2 * LI.entries - 1) : 1;  // 2^kIdxBits >= entries
  static constexpr uint32_t kHiLo = 0x40F80000u;                          // high word of t at j = 0
  static constexpr uint32_t kHiHi = kHiLo + 16u * (uint32_t)((kLut ? LI.entries : 1) - 1) + 15u;
  static constexpr uint32_t kMask = ((1u << kIdxBits) - 1u) << 4;
  static_assert(!kLut || (kIdxBits <= 15 && LI.scale + LI.off < 32768.0), "bucket index inside the high word");

  struct alignas(16) Ent {
    double e;    // E_j, the edge in the bucket domain (+inf past the last edge)
    uint32_t c;  // c_j
    uint32_t pad;
  };
  struct Smem {
    Ent lut[kLut ? LI.entries : 1];
    double edge64[kLut ? 1 : L];
  };

  __device__ static void load(Smem& sm, int tid, int nthreads) {
    if constexpr (kLut) {
      for (int i = tid; i < LI.entries; i += nthreads) {
        const float e = __uint_as_float(pitch_lut_tab[2 * (LI.offset + i)]);
        sm.lut[i].e = __builtin_fma((double)e, LI.scale, kMagic);  // exact; inf stays inf
        sm.lut[i].c = pitch_lut_tab[2 * (LI.offset + i) + 1];
        sm.lut[i].pad = 0u;
      }
    } else {
      constexpr int off = pitch_codebook_offset(ilog2(D), B);
      for (int i = tid; i < L; i += nthreads) sm.edge64[i] = (double)pitch_edge_tab[off + i];
    }
  }

  // Applies f(e, code) to the codes of x[0..N) in order, with u = x * us.
  template <int N, typename F>
  __device__ static void for_codes(const Smem& sm, const double (&x)[N], double us, F&& f) {
    if constexpr (kLut) {
      const double us_m = us * LI.scale;  // exact: LI.scale is a power of two
      typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));  // naturally (16-byte) aligned
      typedef __attribute__((address_space(3))) const u32x4n lds_u32x4;
      typedef __attribute__((address_space(3))) const char lds_byte;
      lds_byte* tab = (lds_byte*)(sm.lut);
#pragma unroll
      for (int b0 = 0; b0 < N; b0 += kBatch) {
        double tt[kBatch];
        double ee[kBatch];
        uint32_t cc[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          if (b0 + i < N) {
            tt[i] = __builtin_fma(x[b0 + i], us_m, kMagic);
            const uint32_t hi = (uint32_t)((uint64_t)__double_as_longlong(tt[i]) >> 32);
            const uint32_t hc = min(max(hi, kHiLo), kHiHi);  // NaN and out-of-table u land on an end bucket
            // one 16-byte read per entry (the offset is a multiple of 16)
            const u32x4n w = *(lds_u32x4*)(tab + (hc & kMask));
            ee[i] = __longlong_as_double((long long)(((uint64_t)w.y << 32) | w.x));
            cc[i] = w.z;
          }
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i)
          if (b0 + i < N) f(b0 + i, cc[i] + (tt[i] > ee[i] ? 1u : 0u));
      }
    } else {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const double u = x[e] * us;
        uint32_t cd = 0;
#pragma unroll
        for (int s = L / 2; s >= 1; s >>= 1) cd = (u > sm.edge64[cd + s - 1]) ? cd + s : cd;
        f(e, cd);
      }
    }
  }

  // Codes of x[0..N) packed into words as they are produced: code e at bits [e*B, e*B + B) of w.
  template <int N, int NWORDS>
  __device__ static void codes_packed(const Smem& sm, const double (&x)[N], double us, uint32_t (&w)[NWORDS]) {
#pragma unroll
    for (int i = 0; i < NWORDS; ++i) w[i] = 0u;
    for_codes(sm, x, us, [&](int e, uint32_t cd) {
      const int pos = e * B, wi = pos >> 5, sh = pos & 31;
      w[wi] |= cd << sh;
      if (sh + B > 32) w[wi + 1] |= cd >> (32 - sh);
    });
  }

  template <int N>
  __device__ static void codes(const Smem& sm, const double (&x)[N], double us, uint32_t (&out)[N]) {
    for_codes(sm, x, us, [&](int e, uint32_t cd) { out[e] = cd; });
  }
};

// TurboQuant quantiser with 8-byte bucket-table entries, for the staged-stage encoder. The bucket domain is
// t = u * 2^m + off + 2^k + 2^(k-1) in [2^k, 2^(k+1)) with k = 20 - log2(R), R the bytes per table row, so
// bits 20 - k .. 19 of t's high word hold the bucket index plus 2^(k-1) and masking them gives the row's byte
// offset directly. An entry is one float64: the bucket's edge E_j mapped to that domain (exact; gen_tables.py
// checks that its low 8 mantissa bits are zero) with c_j stored in those 8 bits, or, past the last edge, the
// largest such value below 2^(k+1). code = c_j + [t > E'_j] comes out of one compare and one add with carry
// of the entry's low word; its bits above B are cleared by the packing. E'_j exceeds E_j by c_j ulps
// (2^-31 bucket units at most), which moves the decision by less than 2^-36 in u, far inside the
// near-boundary band. Tables are replicated (lut8_copies; R = 8 bytes per copy) so that the random lookups of a
// wave conflict on fewer LDS banks.
#ifndef PITCH_LUT8_REP
#define PITCH_LUT8_REP 32  // most copies of a replicated table: lane l reads copy l % REP, so with 32 the 32 lanes an
                           // LDS cycle serves (64 banks of 4 bytes) never share a bank
#endif
#ifndef PITCH_LUT8_STAGED_REP
#define PITCH_LUT8_STAGED_REP 16  // copies of the staged-stage encoder's tables (where they fit)
#endif
#ifndef PITCH_LUT8_REP_MAX
#define PITCH_LUT8_REP_MAX 20480  // largest replicated table in bytes
#endif
// Copies of a table of `bytes`. The staged-stage encoder (d = 64, 128) keeps 16 copies when they fit in
// PITCH_LUT8_REP_MAX bytes and one otherwise: its staging rows leave LDS conflicts that 32 copies do not remove,
// building 32 copies per workgroup cost more than the lookups gained at config-2 and config-4 sizes (medians of
// five runs: -1 to +2.6 %), and more copies of the larger tables cost it a wave per SIMD (2-7 % slower at d = 64,
// b = 6 and 8). The transposed encoder (d >= 256), whose LDS allows it, takes as many copies as fit, up to 32
// (bank conflicts 0.39 -> 0.00 of its LDS cycles at d = 1024, b = 3 and 4).
// The staged-stage encoder's LDS besides its table: the staging rows of its four waves (Hs::WAVES * Hs::ROWS
// float64, checked in hs_run). Its copies are halved until rows and table fit three workgroups per CU (160 KB):
// 16 copies of the d = 128, b = 5 table left room for two.
constexpr int hs_rows_bytes(int D) { return D == 64 ? 41984 : (D == 128 ? 37376 : 0); }
constexpr int kHsLdsBudget = 54528;
constexpr int lut8_copies(int bytes, bool fill, int rows_bytes = 0) {
  if (!fill) {
    int r = PITCH_LUT8_STAGED_REP * bytes <= PITCH_LUT8_REP_MAX ? PITCH_LUT8_STAGED_REP : 1;
    while (r > 1 && rows_bytes + r * bytes + 8 > kHsLdsBudget) r /= 2;
    return r;
  }
  int r = 1;
  while (r < PITCH_LUT8_REP && 2 * r * bytes <= PITCH_LUT8_REP_MAX) r *= 2;
  return r;
}
// (a & m) | b in one v_and_or_b32 (the compiler otherwise splits it into an and and an add).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t b) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(b));
  return r;
}

template <int D, int B>
struct TqLut8 {
  static constexpr int L = 1 << B;
  static constexpr PitchLutInfo LI = pitch_lut_info(ilog2(D), B);
  static constexpr bool kLut = LI.offset >= 0;
  static constexpr int N = kLut ? LI.entries : 1;
  static constexpr int REP = kLut ? lut8_copies(N * 8, D >= 256, hs_rows_bytes(D)) : 1;
  static constexpr int R = 8 * REP;                     // bytes per row
  static constexpr int K = 20 - ilog2(R);               // t in [2^K, 2^(K+1))
  static constexpr double kMagic = double(1 << K) + double(1 << (K - 1)) + LI.off;
  static constexpr int kIdxBits = kLut ? ilog2(2 * N - 1) : 1;  // 2^kIdxBits >= N
  static constexpr uint32_t kHiLo = (uint32_t)(1023 + K) << 20 | 0x80000u;  // high word of 2^K + 2^(K-1)
  static constexpr uint32_t kHiHi = kHiLo + (uint32_t)R * (uint32_t)(N - 1) + (uint32_t)(R - 1);
  static constexpr uint32_t kMask = ((1u << kIdxBits) - 1u) * (uint32_t)R;
  static constexpr uint64_t kTop = ((uint64_t)(1023 + K) << 52) | 0xFFFFFFFFFFF00ull;  // below 2^(K+1), low byte 0
  static_assert(!kLut || (kIdxBits <= K - 1 && LI.scale + LI.off < double(1 << (K - 1))), "index in the high word");
  static_assert(kLut || B >= 7, "every table of B <= 6 fits");

  struct Smem {
    uint64_t tab[kLut ? N * REP : 1];
    double edge64[kLut ? 1 : L];
  };

  // The table set-up of a workgroup of NT threads. Each thread's global loads go out together (the index is
  // clamped instead of tested, so no load sits in a branch) and are waited for once.
  template <int NT>
  __device__ static void load(Smem& sm, int tid) {
    if constexpr (kLut) {
      constexpr int kIt = (N * REP + NT - 1) / NT;
      uint32_t e_bits[kIt], c[kIt];
#pragma unroll
      for (int k = 0; k < kIt; ++k) {
        const int j = min(tid + k * NT, N * REP - 1) / REP;
        e_bits[k] = pitch_lut_tab[2 * (LI.offset + j)];
        c[k] = pitch_lut_tab[2 * (LI.offset + j) + 1];
      }
#pragma unroll
      for (int k = 0; k < kIt; ++k) {
        const int i = tid + k * NT;
        if (i < N * REP) {
          const float e = __uint_as_float(e_bits[k]);
          const uint64_t bits = __builtin_isinf(e) ? kTop : (uint64_t)__double_as_longlong(__builtin_fma((double)e, LI.scale, kMagic));
          sm.tab[i] = bits | c[k];
        }
      }
    } else {
      constexpr int off = pitch_codebook_offset(ilog2(D), B);
      for (int i = tid; i < L; i += NT) sm.edge64[i] = (double)pitch_edge_tab[off + i];
    }
  }

  // Applies f(e, raw) to x[0..NX) in order, with u = x * us; the low B bits of raw are the code of x[e].
  // Lookups are issued in batches of QB (at most 15, what the LDS wait counter tracks) before any is used.
  template <int QB, int NX, typename F>
  __device__ static void for_codes(const Smem& sm, const double (&x)[NX], double us, int lane, F&& f) {
    if constexpr (kLut) {
      const double us_m = us * LI.scale;  // exact: LI.scale is a power of two
      typedef __attribute__((address_space(3))) const uint64_t lds_u64;
      typedef __attribute__((address_space(3))) const char lds_byte;
      lds_byte* tab = (lds_byte*)(sm.tab);
      const uint32_t loff = REP > 1 ? (uint32_t)(lane % REP) * 8u : 0u;
      constexpr int kB = QB;
#pragma unroll
      for (int b0 = 0; b0 < NX; b0 += kB) {
        double tt[kB];
        uint64_t ee[kB];
#pragma unroll
        for (int i = 0; i < kB; ++i) {
          if (b0 + i < NX) {
            tt[i] = __builtin_fma(x[b0 + i], us_m, kMagic);
            const uint32_t hi = (uint32_t)((uint64_t)__double_as_longlong(tt[i]) >> 32);
            const uint32_t hc = min(max(hi, kHiLo), kHiHi);  // NaN and out-of-table u land on an end bucket
            ee[i] = *(lds_u64*)(tab + and_or(hc, kMask, loff));
          }
        }
#pragma unroll
        for (int i = 0; i < kB; ++i)
          if (b0 + i < NX) f(b0 + i, (uint32_t)ee[i] + (tt[i] > __longlong_as_double((long long)ee[i]) ? 1u : 0u));
      }
    } else {
#pragma unroll
      for (int e = 0; e < NX; ++e) {
        const double u = x[e] * us;
        uint32_t cd = 0;
#pragma unroll
        for (int s = L / 2; s >= 1; s >>= 1) cd = (u > sm.edge64[cd + s - 1]) ? cd + s : cd;
        f(e, cd);
      }
    }
  }

  // Codes of x[0..NX) packed into words as they are produced: code e at bits [e*B, e*B + B) of w. Each word
  // is a shift register: v_alignbit(raw, w, s) shifts w down by s and brings the low s bits of raw in at the
  // top (raw's bits above s are dropped), so a word ends up holding the last 32 bits shifted into it, the
  // earliest at bit 0. A code that straddles two words is shifted into both: its low 32 - sh bits end the
  // first, and all B bits go into the second, whose remaining codes push the low ones out again. When the
  // codes end part-way into the last word, they sit in its top bits and one shift moves them down. One
  // instruction per code, where masking and or-ing takes two.
  template <int QB, int NX, int NWORDS>
  __device__ static void codes_packed(const Smem& sm, const double (&x)[NX], double us, int lane,
                                      uint32_t (&w)[NWORDS]) {
    static_assert(NWORDS * 32 >= NX * B, "room for every code");
#pragma unroll
    for (int i = 0; i < NWORDS; ++i) w[i] = 0u;
    for_codes<QB>(sm, x, us, lane, [&](int e, uint32_t raw) {
      const int pos = e * B, wi = pos >> 5, sh = pos & 31;
      if (sh + B > 32) {
        w[wi] = __builtin_amdgcn_alignbit(raw, w[wi], 32 - sh);
        w[wi + 1] = __builtin_amdgcn_alignbit(raw, w[wi + 1], B);
      } else {
        w[wi] = __builtin_amdgcn_alignbit(raw, w[wi], B);
      }
    });
    constexpr int kRem = (NX * B) & 31;
    if constexpr (kRem != 0) w[(NX * B) >> 5] >>= 32 - kRem;
  }
};

#ifndef PITCH_NT_STORE
#define PITCH_NT_STORE 1  // decoded vectors are streamed out with nontemporal stores (0: regular stores)
#endif

// ----------------------------------------------------------------------------------------------------
#ifndef PITCH_VEC_ENC_NT
#define PITCH_VEC_ENC_NT 1  // the team encoder reads its input with non-temporal loads
#endif
#ifndef PITCH_POLAR_WAVES
#define PITCH_POLAR_WAVES 1  // minimum waves per SIMD requested for the team encoder (caps its VGPRs)
#endif
// The team encoder's work on one segment: count vectors from in to codes_out / scales_out, blocks of VPB vectors
// from vector first on, stride vectors apart. p supplies the rotation signs and the key-bias tables.
template <int D, int B, bool POLAR, int IO, bool KBIAS>
__device__ __forceinline__ void vec_encode_run(const VecArgs& p, const void* in, uint32_t* codes_out,
                                               float* scales_out, uint64_t count, uint64_t first, uint64_t stride) {
  using G = Geom<D>;
  constexpr int L = 1 << B;
  constexpr int NW = (D * B + 31) / 32;  // 32-bit words of codes per vector
  constexpr bool kStage = D >= 32;       // codes are packed from LDS in groups of 32
  using Q = TqQuant<D, B>;
  __shared__ typename Q::Smem s_q;
  // staged code bytes: one row of D / 4 + 4 words per vector, so the team lanes of consecutive vectors write
  // to different LDS banks and every 32-code group stays 16-byte aligned
  constexpr int kStageRow = D / 4 + 4;
  __shared__ __attribute__((aligned(16))) uint32_t s_stage[kStage ? G::VPB * kStageRow : 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int t = lane & (G::T - 1);
  const int slot = (tid >> 6) * G::V + lane / G::T;

  if constexpr (!POLAR) Q::load(s_q, tid, kBlock);
  const uint32_t fbits = p.lane_flips[t];
  uint32_t flip[G::E];
#pragma unroll
  for (int e = 0; e < G::E; ++e) flip[e] = ((fbits >> e) & 1u) << 31;
  __syncthreads();

  // Full iterations run without bounds checks; in the last, partial one, lanes past the end re-read the
  // last vector (loads stay unconditional) and store nothing.
  auto body = [&](uint64_t base, auto tail_c) {
    constexpr bool TAIL = decltype(tail_c)::value;
    const uint64_t v = base + slot;
    const bool valid = !TAIL || v < count;
    const uint64_t row = (valid ? v : count - 1) * D;

    // load every chunk before converting (all loads in flight together), then apply the signs (exact)
    float f[G::E];
#pragma unroll
    for (int k = 0; k < G::CH; ++k) {
      if constexpr (PITCH_VEC_ENC_NT && G::W == 4)  // read-once input: streamed past the caches
        load4_nt<IO>(in, row + G::W * (k * G::T + t), *(float(*)[G::W])(f + k * G::W));
      else
        load_elems<IO, G::W>(in, row + G::W * (k * G::T + t), *(float(*)[G::W])(f + k * G::W));
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KBIAS) {  // key-bias removal: encode x - o (mechanism_eval.py:113-116)
#pragma unroll
      for (int k = 0; k < G::CH; ++k) {
        float o[G::W];
        key_bias_offset<D, G::W>(p, valid ? v : count - 1, G::W * (k * G::T + t), o);
#pragma unroll
        for (int r = 0; r < G::W; ++r) f[k * G::W + r] = f[k * G::W + r] - o[r];
      }
    }
    double x[G::E];
#pragma unroll
    for (int e = 0; e < G::E; ++e) x[e] = (double)__uint_as_float(__float_as_uint(f[e]) ^ flip[e]);
    float scale;
    uint32_t code[G::E];
    if constexpr (!POLAR) {
      // u = H(s * x) / (||x|| sqrt(d)) (pitch_reference.py:96-98): the transform runs on the unscaled
      // input and one multiply by RN(RN(1 / norm) / sqrt(d)) follows; u differs from the reference's
      // divide-first order by a few float64 ulps, far inside the near-boundary band.
      double ss = 0.0;
#pragma unroll
      for (int e = 0; e < G::E; ++e) ss = __builtin_fma(x[e], x[e], ss);
      ss = team_reduce<G::T>(ss, [](double a, double b) { return a + b; });
      const double nrm = __builtin_sqrt(ss);
      const double safe = nrm > 0.0 ? nrm : 1.0;
      const double us = (1.0 / safe) * DimConst<D>::kInvSqrt;
      scale = (float)nrm;
      fwht<D, double>(x, t);
      Q::codes(s_q, x, us, code);
    } else {
      // The codes depend only on the directions and the radii relative to rmax, which the division by sqrt(d)
      // of rotate() leaves unchanged (up to float64 rounding, far inside the near-boundary band): the pairs are
      // taken from the unnormalised transform and only rmax is scaled (exactly when d is a power of 4).
      fwht<D, double>(x, t);
      // pairs (y_2p, y_2p+1) -> radius and angle (pitch_reference.py:111-121)
      constexpr int NP = G::E / 2;
      double r2[NP];
      double rmax2 = 0.0;
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        const double a = x[2 * q], c = x[2 * q + 1];
        r2[q] = __builtin_fma(a, a, c * c);
        rmax2 = r2[q] > rmax2 ? r2[q] : rmax2;
      }
      rmax2 = team_reduce<G::T>(rmax2, [](double a, double b) { return a > b ? a : b; });
      const double rmax = __builtin_sqrt(rmax2);  // = max of the pairs' radii: sqrt is monotone
      const double safe = rmax > 0.0 ? rmax : 1.0;
      const double inv = 1.0 / safe;
      uint32_t need = 0u;  // bit q: pair q is decided by the float64 path
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        // float32 fast path on the pair scaled by 1 / rmax (no overflow or underflow of its square)
        const float af = (float)(x[2 * q] * inv), cf = (float)(x[2 * q + 1] * inv);
        const float rf = __builtin_amdgcn_sqrtf(__builtin_fmaf(af, af, cf * cf));
        bool ok = r2[q] > 0.0;
        const float kr = guarded_floor(__builtin_fmaf(rf, float(L - 1), 0.5f), ok);
        const float ka = guarded_floor(__builtin_fmaf(angle_turns<B>(cf, af), float(L), 0.5f), ok);
        code[2 * q] = (uint32_t)__builtin_fminf(kr, float(L - 1));
        code[2 * q + 1] = (uint32_t)ka & (uint32_t)(L - 1);
        need |= ok ? 0u : 1u << q;
      }
      // float64 path for the pairs the guard rejected (rare): one shared out-of-line copy
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        if (need & (1u << q)) {
          const uint2 cc = polar_codes_exact<B>(x[2 * q], x[2 * q + 1], r2[q], safe);
          code[2 * q] = cc.x;
          code[2 * q + 1] = cc.y;
        }
      }
      scale = (float)div_sqrt_d<D>(rmax);
    }

    if constexpr (kStage) {
#pragma unroll
      for (int k = 0; k < G::CH; ++k) {
        const int c0 = G::W * (k * G::T + t);
        s_stage[slot * kStageRow + (c0 >> 2)] = code[4 * k] | (code[4 * k + 1] << 8) | (code[4 * k + 2] << 16) |
                                        (code[4 * k + 3] << 24);
      }
    } else {
      // one lane owns the whole vector: pack in registers (element e is coordinate e)
      uint32_t w[NW];
#pragma unroll
      for (int i = 0; i < NW; ++i) w[i] = 0u;
#pragma unroll
      for (int i = 0; i < D; ++i) {
        const int pos = i * B, wi = pos >> 5, sh = pos & 31;
        w[wi] |= code[i] << sh;
        if (sh + B > 32) w[wi + 1] |= code[i] >> (32 - sh);
      }
      if (valid) store_words<NW>(codes_out + v * NW, w);
    }
    if (t == 0 && valid) scales_out[v] = scale;

    if constexpr (kStage) {
      __syncthreads();
      constexpr int GPV = D / 32;  // 32-code groups per vector; each packs into exactly B words
      constexpr int NG = G::VPB * GPV;
#pragma unroll
      for (int g0 = 0; g0 < NG; g0 += kBlock) {
        const int g = g0 + tid;
        if (NG % kBlock == 0 || g < NG) {
          const int vs = g / GPV, gi = g % GPV;
          const uint64_t vv = base + vs;
          if (!TAIL || vv < count) {
            const uint4* q = (const uint4*)(s_stage + vs * kStageRow + 8 * gi);
            const uint4 q0 = q[0], q1 = q[1];
            const uint32_t bytes[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            uint32_t w[B];
            pack32<B>(bytes, w);
            store_words<B>(codes_out + vv * NW + gi * B, w);
          }
        }
      }
      __syncthreads();
    }
  };
  for (uint64_t base = first; base < count; base += stride) {
    if (base + G::VPB <= count) body(base, std::false_type{});
    else body(base, std::true_type{});
  }
}

template <int D, int B, bool POLAR, int IO, bool KBIAS>
__global__ __launch_bounds__(kBlock, PITCH_POLAR_WAVES) void vec_encode(VecArgs p) {
  vec_encode_run<D, B, POLAR, IO, KBIAS>(p, p.in, p.codes_out, p.scales_out, p.count,
                                         (uint64_t)blockIdx.x * Geom<D>::VPB, (uint64_t)gridDim.x * Geom<D>::VPB);
}

// A batch of independent segments with one configuration in one launch (pitch_enqueue_encode_batch): the blocks
// [block_start[i], block_start[i + 1]) encode segment i. Each encoder below has such a batched form, and a batch
// runs the one a single call of its configuration runs (enc_kind), so both write the same bytes.
template <int D, int B, bool POLAR, int IO>
__global__ __launch_bounds__(kBlock, PITCH_POLAR_WAVES) void vec_encode_batch(VecBatchArgs pb) {
  const BatchSlot s = batch_slot(pb);
  vec_encode_run<D, B, POLAR, IO, false>(pb.common, s.seg.in, s.seg.codes_out, s.seg.scales_out, s.seg.count,
                                         s.block * Geom<D>::VPB, s.blocks * Geom<D>::VPB);
}

// ----------------------------------------------------------------------------------------------------
// Decode tables in LDS. Codes are looked up several at a time: a chunk of 4 TurboQuant 2-bit codes indexes a
// 256-entry table of float4, pairs of codes (TurboQuant 3..5 bits; PolarQuant (radius, angle) for up to 5
// bits) index a 2^(2b)-entry table of float2; wider codes are looked up one at a time.
template <int B, bool POLAR, int W>
struct DecTab {
  static constexpr int L = 1 << B;
  static constexpr int G = W < 4 ? (B <= 5 ? 2 : 1) : (POLAR ? (B <= 5 ? 2 : 1) : (B == 2 ? 4 : (B <= 5 ? 2 : 1)));
  static constexpr int ENTRIES = G == 4 ? 256 : (G == 2 ? (1 << (2 * B)) : L);
  static constexpr int FLOATS = G == 1 ? (POLAR ? 3 * L : L) : ENTRIES * G;
  // transform stages folded into the table: an entry of G consecutive coordinates holds their values after
  // the butterflies on coordinate bits 0 .. log2(G) - 1, the first stages of the transform
  static constexpr int PRE = G == 4 ? 2 : (G == 2 ? 1 : 0);
};

// The decode table is built in two steps so that a kernel can issue its first code loads between them: the table's
// source values are loaded first (load_dec_table), the entries are computed and written to LDS after
// (write_dec_table). Loads complete in order, so waiting for the source values then leaves the code loads in flight.
template <int D, int B, bool POLAR>
struct DecTabSrc {
  using TB = DecTab<B, POLAR, Geom<D>::W>;
  static constexpr int ENTRIES = TB::G == 1 ? TB::L : TB::ENTRIES;  // entries (or table rows) built per call
  static constexpr int R = (ENTRIES + kBlock - 1) / kBlock;         // entries per thread
  static constexpr int S = POLAR ? 3 : (TB::G == 4 ? 4 : (TB::G == 2 ? 2 : 1));  // source values per entry
  float v[R][S];
};

template <int D, int B, bool POLAR>
__device__ __forceinline__ DecTabSrc<D, B, POLAR> load_dec_table() {
  using TB = DecTab<B, POLAR, Geom<D>::W>;
  using Src = DecTabSrc<D, B, POLAR>;
  constexpr int L = TB::L;
  Src src;
  // Threads past the last entry build the last entry again (the same value to the same place), so loads and writes
  // are unconditional and the loads stay where they are written, ahead of the caller's next loads.
#pragma unroll
  for (int r = 0; r < Src::R; ++r) {
    const int i = threadIdx.x + r * kBlock;
    const int ic = i < Src::ENTRIES ? i : Src::ENTRIES - 1;
    if constexpr (POLAR) {
      constexpr int off = pitch_polar_offset(B);
      const int ir = TB::G == 2 ? (ic & (L - 1)) : ic, ia = TB::G == 2 ? (ic >> B) : ic;
      src.v[r][0] = pitch_polar_radius_tab[off + ir];
      src.v[r][1] = pitch_polar_cos_tab[off + ia];
      src.v[r][2] = pitch_polar_sin_tab[off + ia];
    } else {
      const float* cb = pitch_codebook_tab + pitch_codebook_offset(ilog2(D), B);
      if constexpr (TB::G == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) src.v[r][j] = cb[(ic >> (2 * j)) & 3];
      } else if constexpr (TB::G == 2) {
        src.v[r][0] = cb[ic & (L - 1)];
        src.v[r][1] = cb[ic >> B];
      } else {
        src.v[r][0] = cb[ic];
      }
    }
  }
  return src;
}

template <int D, int B, bool POLAR>
__device__ __forceinline__ void write_dec_table(const DecTabSrc<D, B, POLAR>& src, float* s_tab) {
  using TB = DecTab<B, POLAR, Geom<D>::W>;
  using Src = DecTabSrc<D, B, POLAR>;
  constexpr int L = TB::L;
#pragma unroll
  for (int r = 0; r < Src::R; ++r) {
    const int i0 = threadIdx.x + r * kBlock;
    const int i = i0 < Src::ENTRIES ? i0 : Src::ENTRIES - 1;
    if constexpr (POLAR) {
      const float rr = src.v[r][0];
      if constexpr (TB::G == 2) {
        const float x = rr * src.v[r][1], y = rr * src.v[r][2];
        s_tab[2 * i] = x + y;
        s_tab[2 * i + 1] = x - y;
      } else {
        s_tab[i] = rr;
        s_tab[L + i] = src.v[r][1];
        s_tab[2 * L + i] = src.v[r][2];
      }
    } else if constexpr (TB::G == 4) {
      const float q0 = src.v[r][0], q1 = src.v[r][1], q2 = src.v[r][2], q3 = src.v[r][3];
      const float a0 = q0 + q1, a1 = q0 - q1, a2 = q2 + q3, a3 = q2 - q3;
      s_tab[4 * i] = a0 + a2;
      s_tab[4 * i + 1] = a1 + a3;
      s_tab[4 * i + 2] = a0 - a2;
      s_tab[4 * i + 3] = a1 - a3;
    } else if constexpr (TB::G == 2) {
      const float x = src.v[r][0], y = src.v[r][1];
      s_tab[2 * i] = x + y;
      s_tab[2 * i + 1] = x - y;
    } else {
      s_tab[i] = src.v[r][0];
    }
  }
}

// Unpacks the W codes of one chunk (bits [0, W*B) of `bits`) into W rotated-domain values, with the first
// DecTab::PRE transform stages already applied.
template <int D, int B, bool POLAR>
__device__ __forceinline__ void decode_chunk(uint32_t bits, const float* s_tab, float* y) {
  using TB = DecTab<B, POLAR, Geom<D>::W>;
  constexpr int W = Geom<D>::W, L = TB::L;
  if constexpr (TB::G == 4) {
    const float4 q = ((const float4*)s_tab)[bits & 0xFFu];
    y[0] = q.x; y[1] = q.y; y[2] = q.z; y[3] = q.w;
  } else if constexpr (TB::G == 2) {
#pragma unroll
    for (int pr = 0; pr < W / 2; ++pr) {
      const float2 q = ((const float2*)s_tab)[(bits >> (2 * B * pr)) & ((1u << (2 * B)) - 1u)];
      y[2 * pr] = q.x;
      y[2 * pr + 1] = q.y;
    }
  } else if constexpr (POLAR) {
#pragma unroll
    for (int r = 0; r < W; r += 2) {
      const uint32_t cr = (bits >> (B * r)) & (L - 1);
      const uint32_t ca = (bits >> (B * (r + 1))) & (L - 1);
      const float rr = s_tab[cr];
      y[r] = rr * s_tab[L + ca];
      y[r + 1] = rr * s_tab[2 * L + ca];
    }
  } else {
#pragma unroll
    for (int r = 0; r < W; ++r) y[r] = s_tab[(bits >> (B * r)) & (L - 1)];
  }
}

// The last step of every per-vector decoder: x = s * (H y) * scale / sqrt(d). y comes from fwht_f32_lane_signed,
// equal to the transform up to the lane's sign (lane_sign) and, for a zero, up to the sign of that zero, which
// differs between lane layouts. dec_scale folds the lane's sign into the vector's factor; dec_out multiplies by it
// with an fma whose addend is +0, which gives every exact zero the sign +0 (RN(-0 + +0) = +0) and every other
// value RN(y * f), then applies the coordinate's random sign. So each decoder, whatever its lane layout, writes
// the same bytes for the same codes: a zero of the transform decodes to +0 with the coordinate's sign applied,
// as the reference's wht(y) * signs gives for a transform zero of +0 (pitch_reference.py:34).
template <int D>
__device__ __forceinline__ float dec_scale(float scale, uint32_t lane_sign) {
  return __uint_as_float(__float_as_uint(scale * DimConst<D>::kInvSqrtF) ^ lane_sign);
}
__device__ __forceinline__ float dec_out(float y, float f, uint32_t sign) {
  return __uint_as_float(__float_as_uint(__builtin_fmaf(y, f, 0.0f)) ^ sign);
}

#ifndef PITCH_DEC_LDS_STORE
#define PITCH_DEC_LDS_STORE 1  // decoded vectors are staged in LDS and stored as contiguous wave blocks
#endif

#ifndef PITCH_DEC_PAD
#define PITCH_DEC_PAD 16  // floats of padding per vector in the decoders' LDS output staging
#endif
#ifndef PITCH_DEC_WAVES
#define PITCH_DEC_WAVES 1  // minimum waves per SIMD requested for the decoders (caps their VGPRs)
#endif
#ifndef PITCH_DEC_ONE_PER_WG_MIN
#define PITCH_DEC_ONE_PER_WG_MIN (64ull << 20)  // float32 decodes writing [MIN, MAX) bytes: one workgroup per block
#endif
#ifndef PITCH_DEC_ONE_PER_WG_MAX
#define PITCH_DEC_ONE_PER_WG_MAX (1ull << 62)
#endif
#ifndef PITCH_DEC_WAVE_BASE
#define PITCH_DEC_WAVE_BASE 1  // calls of at least one wave's vectors store from a wave-uniform base
#endif
// Streaming decodes of codes up to PITCH_STREAM_CAP_BITS wide run one launch of every block, held at
// PITCH_STREAM_WG_PER_CU resident workgroups per CU by dynamic LDS; wider codes run launches of one round at the
// kernel's full 8 per CU. d = 1024, 2^19 / 2^21 vectors, % of peak in interleaved repeats (identical bytes), rounds
// -> one launch at 5 per CU: TurboQuant b = 2 66 / 66 -> 72 / 75, b = 3 68 / 65 -> 79 / 74, b = 4 70 / 69 -> 79 / 77,
// b = 5 70 / 69.5 -> 75 / 69.5, b = 6 70 / 68 -> 76 / 71.5, b = 8 73 / 73.5 -> 69 / 67.5; PolarQuant b = 3 68.5 / 66
// -> 81 / 74, b = 4 70 / 69.5 -> 80.5 / 77, b = 6 69 / 66.5 -> 73 / 72. One launch at 3, 4, 6, 7 and 8 per CU was
// slower than at 5 for most widths (b = 8 at 4 per CU: 76 / 72.5).
#ifndef PITCH_STREAM_WG_PER_CU
#define PITCH_STREAM_WG_PER_CU 5
#endif
#ifndef PITCH_STREAM_CAP_BITS
#define PITCH_STREAM_CAP_BITS 6
#endif

// The body of every per-vector decode: count vectors from codes_in / scales_in to out (p supplies the sign masks and
// the key bias), with this workgroup block of nblocks striding over the call.
template <int D, int B, bool POLAR, int IO, bool KBIAS>
__device__ __forceinline__ void vec_decode_run(const VecArgs& p, const uint32_t* codes_in, const float* scales_in,
                                               void* out, uint64_t count, uint64_t block, uint64_t nblocks) {
  using G = Geom<D>;
  using TB = DecTab<B, POLAR, G::W>;
  constexpr int NW = (D * B + 31) / 32;
  constexpr int CB = G::W * B;  // bits of codes per chunk (<= 32)
  __shared__ __attribute__((aligned(16))) float s_tab[TB::FLOATS];
  // optional LDS staging of the output (D >= 64): each wave writes its vectors back contiguously
  constexpr bool kLdsStore = PITCH_DEC_LDS_STORE && D >= 64 && G::W == 4;
  // floats per staged vector: the 16-float padding puts the team lanes of neighbouring vectors, which write
  // in the same LDS cycle, on disjoint banks
  constexpr int kVecStride = D + PITCH_DEC_PAD;
  constexpr int kWaveOutFloats = G::V * kVecStride;
  __shared__ __attribute__((aligned(16))) float s_out[kLdsStore ? 4 * kWaveOutFloats : 4];

  // per wave, the codes (V * NW words) and scales of its V vectors, loaded coalesced and read back per lane
  constexpr int kWaveCodeWords = G::V * NW;
  constexpr int NPL = (kWaveCodeWords + 63) / 64;  // code words each lane loads per batch
  __shared__ uint32_t s_codes[kBlock / 64][kWaveCodeWords];
  __shared__ float s_scale[kBlock / 64][G::V];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int t = lane & (G::T - 1);
  const int wave = tid >> 6, vw = lane / G::T;  // vector of this lane's team within the wave

  const uint32_t fbits = p.lane_flips[t];
  // the transform's lane sign (fwht_f32_lane_signed) is folded into the scale factor (dec_scale), the random
  // signs are applied to the scaled values
  const uint32_t lane_sign = dpp_lane_sign_bit<D>(t);
  uint32_t flip[G::E];
#pragma unroll
  for (int e = 0; e < G::E; ++e) flip[e] = ((fbits >> e) & 1u) << 31;
  // word index and bit offset of each of this lane's chunks (the next word is read when a chunk straddles)
  int wlo[G::CH], whi[G::CH];
  uint32_t wsh[G::CH];
#pragma unroll
  for (int k = 0; k < G::CH; ++k) {
    const int pos = CB * (k * G::T + t);
    wlo[k] = pos >> 5;
    wsh[k] = (uint32_t)(pos & 31);
    whi[k] = ((pos & 31) + CB > 32) ? wlo[k] + 1 : wlo[k];
  }

  // Software pipeline: the codes and scales of the next iteration are loaded before the current one is
  // transformed, so every wave keeps a batch of loads in flight while it computes. A wave loads the contiguous code
  // words of its V vectors with coalesced loads (NPL per lane; per-lane loads of each chunk's own words measured
  // 15 % slower at a 17 GB footprint), stages them in LDS and each lane reads its chunks back. Loads and stores are
  // unconditional: a wave whose vectors run past the end takes the last V vectors instead (the whole call when it
  // has fewer), so it decodes and writes the same bytes to the same places as the wave that owns them. With a
  // fixed number of memory operations per iteration the compiler waits for the next batch's loads without waiting
  // for the previous iteration's stores (gfx9 counts loads and stores together, in order).
  struct Batch {
    uint32_t w[NPL];
    float scale;
    uint64_t wb;  // first vector of the wave's block
  };
  auto fetch = [&](uint64_t base) {
    Batch b;
    const uint64_t nominal = base + (uint64_t)wave * G::V;
    b.wb = count >= (uint64_t)G::V ? (nominal < count - G::V ? nominal : count - G::V) : 0;
    const uint32_t* cw = codes_in + b.wb * NW;
    // in a call of fewer than V vectors, words past the call's last one read the last word (never used)
    const uint64_t last = count * NW - 1 - b.wb * NW;
#pragma unroll
    for (int m = 0; m < NPL; ++m) {
      const uint64_t i = (uint64_t)(lane + 64 * m < kWaveCodeWords ? lane + 64 * m : kWaveCodeWords - 1);
      b.w[m] = cw[i < last ? i : last];
    }
    const uint64_t vs = b.wb + (uint64_t)(lane % G::V);
    b.scale = scales_in[vs < count ? vs : count - 1];
    return b;
  };
  // the team's vector within the wave's block: vw, or the call's last vector for teams past the end (only in a
  // call of fewer than V vectors)
  auto local_vector = [&](const Batch& b) -> int {
    const uint64_t lastv = count - 1 - b.wb;
    return (uint64_t)vw < lastv ? vw : (int)lastv;
  };
  // stage the batch in LDS, read the lane's chunks back, table lookups and the transform
  auto transform = [&](const Batch& b, float (&y)[G::E], float& scale) {
#pragma unroll
    for (int m = 0; m < NPL; ++m) {
      const int i = lane + 64 * m < kWaveCodeWords ? lane + 64 * m : kWaveCodeWords - 1;
      s_codes[wave][i] = b.w[m];
    }
    if (lane < G::V) s_scale[wave][lane] = b.scale;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int lv = local_vector(b);
    const uint32_t* row = s_codes[wave] + lv * NW;
    scale = s_scale[wave][lv];
#pragma unroll
    for (int k = 0; k < G::CH; ++k)
      decode_chunk<D, B, POLAR>(__builtin_amdgcn_alignbit(row[whi[k]], row[wlo[k]], wsh[k]), s_tab, y + k * G::W);
    fwht_f32_lane_signed<D, TB::PRE>(y, t);
  };
  auto body = [&](const Batch& b, float (&y)[G::E], float scale) {
    const uint64_t v = b.wb + (uint64_t)local_vector(b);
    const float f = dec_scale<D>(scale, lane_sign);
    if constexpr (kLdsStore) {
      // stage the wave's vectors in LDS, then write them back as contiguous 1 KB wave stores
      float* ws = s_out + (tid >> 6) * kWaveOutFloats;
#pragma unroll
      for (int k = 0; k < G::CH; ++k) {
        float o[G::W];
#pragma unroll
        for (int r = 0; r < G::W; ++r)
          o[r] = dec_out(y[k * G::W + r], f, flip[k * G::W + r]);
        *(float4*)(ws + vw * kVecStride + G::W * (k * G::T + t)) = float4{o[0], o[1], o[2], o[3]};
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint64_t wbase = b.wb;  // first vector of this wave
      constexpr int K = Io<IO>::kPerChunk;  // elements per 16-byte store
      static_assert((G::V * D) % (64 * K) == 0, "whole 16-byte stores per lane");
      if constexpr (PITCH_DEC_WAVE_BASE && !KBIAS) {
        // The wave's output is one contiguous run from its first vector: a wave-uniform base and the lane's 16-byte
        // offsets. Fetch clamps the first vector to count - V, so the run lies inside the call except in a call of
        // fewer than V vectors, whose chunks past the end are not stored.
        const uint64_t wb_u = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(wbase >> 32)) << 32) |
                              __builtin_amdgcn_readfirstlane((uint32_t)wbase);
        const uint64_t left = count - wb_u;  // vectors of the call from the wave's first one on
        char* wout = (char*)out + wb_u * (uint64_t)D * Io<IO>::kBytes;
        // 16-byte chunk q = lane + 64 m of the wave's output: LDS row q / CPV at chunk q % CPV, written to byte 16 q;
        // both are the lane's base plus a constant per m
        constexpr int CPV = D / K;  // 16-byte chunks per vector
        static_assert(CPV <= 64 ? 64 % CPV == 0 : CPV % 64 == 0, "chunks per vector divide or are divided by 64");
        const float* lp = CPV <= 64 ? ws + (lane / CPV) * kVecStride + K * (lane % CPV) : ws + K * lane;
        char* sp = wout + 16 * lane;
#pragma unroll
        for (int m = 0; m < G::V * D / K / 64; ++m) {
          const int off = CPV <= 64 ? m * (64 / CPV) * kVecStride
                                    : (m / (CPV / 64)) * kVecStride + 64 * K * (m % (CPV / 64));
          const int vq = CPV <= 64 ? lane / CPV + m * (64 / CPV) : m / (CPV / 64);  // the chunk's vector
          float o[K];
#pragma unroll
          for (int h = 0; h < K / 4; ++h) {
            const float4 val = *(const float4*)(lp + off + 4 * h);
            o[4 * h] = val.x; o[4 * h + 1] = val.y; o[4 * h + 2] = val.z; o[4 * h + 3] = val.w;
          }
          if ((uint64_t)vq < left) store_elems<IO, K>(sp + 1024 * m, 0, o, PITCH_NT_STORE);
        }
        __builtin_amdgcn_wave_barrier();
        return;
      }
#pragma unroll
      for (int m = 0; m < G::V * D / K / 64; ++m) {
        const int q = lane + 64 * m;          // 16-byte chunk of the wave's output block
        const int vq = q / (D / K), cq = q % (D / K);
        float o[K];
#pragma unroll
        for (int h = 0; h < K / 4; ++h) {
          const float4 val = *(const float4*)(ws + vq * kVecStride + K * cq + 4 * h);
          o[4 * h] = val.x; o[4 * h + 1] = val.y; o[4 * h + 2] = val.z; o[4 * h + 3] = val.w;
        }
        if constexpr (KBIAS) {  // key-bias removal: restore x + o (mechanism_eval.py:113-116)
          float ob[K];
          const uint64_t vv = wbase + vq < count ? wbase + vq : count - 1;
          key_bias_offset<D, K>(p, vv, K * cq, ob);
#pragma unroll
          for (int r = 0; r < K; ++r) o[r] = o[r] + ob[r];
        }
        const uint64_t vd = wbase + vq < count ? wbase + vq : count - 1;
        store_elems<IO, K>(out, vd * D + (uint64_t)K * cq, o, PITCH_NT_STORE);
      }
      __builtin_amdgcn_wave_barrier();
    } else {
#pragma unroll
      for (int k = 0; k < G::CH; ++k) {
        float o[G::W];
#pragma unroll
        for (int r = 0; r < G::W; ++r)
          o[r] = dec_out(y[k * G::W + r], f, flip[k * G::W + r]);
        if constexpr (KBIAS) {
          float ob[G::W];
          key_bias_offset<D, G::W>(p, v, G::W * (k * G::T + t), ob);
#pragma unroll
          for (int r = 0; r < G::W; ++r) o[r] = o[r] + ob[r];
        }
        store_elems<IO, G::W>(out, v * D + G::W * (k * G::T + t), o, PITCH_NT_STORE);
      }
    }
  };
  // Two batches alternate (no register copies of batches that may still be in flight), and the loop is
  // rotated so that each batch is waited for in straight-line code after exactly one iteration's stores and the
  // next batch's loads: fetch A(i), fetch B(i + 1), compute A(i); then fetch A(i + 2), compute B(i + 1),
  // fetch B(i + 3), compute A(i + 2), ...
  const uint64_t stride = nblocks * G::VPB;
  uint64_t base = block * G::VPB;
  auto compute = [&](const Batch& b, uint64_t) {
    float y[G::E];
    float scale;
    transform(b, y, scale);
    body(b, y, scale);
  };
  // The first two batches are requested before the decode table is built, so their latency overlaps the table's
  // (a short launch pays one memory latency before its first stores instead of two); the barrier that publishes
  // the table orders LDS only and leaves these loads in flight.
  const auto tab_src = load_dec_table<D, B, POLAR>();
  __builtin_amdgcn_sched_barrier(0);
  Batch ba = fetch(base);
  Batch bb = fetch(base + stride);
  write_dec_table<D, B, POLAR>(tab_src, s_tab);
  asm volatile("" ::"v"(fbits));  // the sign word (loaded before the batches) is waited for here, not after them
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (base >= count) return;  // uniform per workgroup; no barrier follows
  compute(ba, base);
  for (;;) {
    base += stride;
    if (base >= count) break;
    ba = fetch(base + stride);
    __builtin_amdgcn_sched_barrier(0);
    compute(bb, base);
    __builtin_amdgcn_sched_barrier(0);
    base += stride;
    if (base >= count) break;
    bb = fetch(base + stride);
    __builtin_amdgcn_sched_barrier(0);
    compute(ba, base);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int D, int B, bool POLAR, int IO, bool KBIAS>
__global__ __launch_bounds__(kBlock, PITCH_DEC_WAVES) void vec_decode(VecArgs p) {
  vec_decode_run<D, B, POLAR, IO, KBIAS>(p, p.codes_in, p.scales_in, p.out, p.count, blockIdx.x, gridDim.x);
}

// A batch of independent segments with one configuration in one launch (pitch_enqueue_decode_batch): the blocks
// [block_start[i], block_start[i + 1]) decode segment i with the body of a single call, so a batch writes the bytes
// the single calls write (the streaming decoder, which long float32 calls take, writes the same bytes as this one).
template <int D, int B, bool POLAR, int IO>
__global__ __launch_bounds__(kBlock, PITCH_DEC_WAVES) void vec_decode_batch(DecBatchArgs pb) {
  const uint32_t i = batch_item(pb);
  vec_decode_run<D, B, POLAR, IO, false>(pb.common, pb.codes_in[i], pb.scales_in[i], pb.out[i], pb.count[i],
                                         blockIdx.x - pb.block_start[i], pb.block_start[i + 1] - pb.block_start[i]);
}

// Per-team-lane sign bits for the seed (cached per thread for the last seed).
template <int D, int EE = default_lane_coords(D)>
void fill_lane_flips(uint32_t seed, uint32_t* out) {
  using G = Geom<D, EE>;
  thread_local uint32_t cached_seed = 0;
  thread_local bool have = false;
  thread_local uint32_t cached[32];
  if (!have || cached_seed != seed) {
    for (int t = 0; t < 32; ++t) {
      uint32_t bits = 0;
      if (t < G::T)
        for (int e = 0; e < G::E; ++e)
          if (sign_is_negative(seed, (uint32_t)G::coord(t, e))) bits |= 1u << e;
      cached[t] = bits;
    }
    cached_seed = seed;
    have = true;
  }
  for (int t = 0; t < 32; ++t) out[t] = cached[t];
}

// Rotation-sign masks of the streaming decoder (16 coordinates per lane): fill_lane_flips for teams of up to 32
// lanes; for a team of 64, lane t's 16 bits are bits 16 (t & 1) .. of word t / 2.
template <int D>
void fill_stream_flips(uint32_t seed, uint32_t* out) {
  using G = Geom<D, 16>;
  if constexpr (G::T <= 32) {
    fill_lane_flips<D, 16>(seed, out);
  } else {
    static_assert(G::T == 64 && G::E == 16, "two lanes per mask word");
    thread_local uint32_t cached_seed = 0;
    thread_local bool have = false;
    thread_local uint32_t cached[32];
    if (!have || cached_seed != seed) {
      for (int j = 0; j < 32; ++j) cached[j] = 0u;
      for (int t = 0; t < 64; ++t)
        for (int e = 0; e < 16; ++e)
          if (sign_is_negative(seed, (uint32_t)G::coord(t, e))) cached[t >> 1] |= 1u << (16 * (t & 1) + e);
      cached_seed = seed;
      have = true;
    }
    for (int j = 0; j < 32; ++j) out[j] = cached[j];
  }
}

// ----------------------------------------------------------------------------------------------------
// Streaming decoder for long float32 calls at D = 1024 (the layout also serves D = 128, where vec_decode with one
// workgroup per block is as fast or faster and is used instead). At a footprint of many GB a persistent decoder runs
// at ~5.0 TB/s, while a write stream with the same 10 % of reads reaches ~6 TB/s when the GPU holds 8 workgroups per
// CU, each wave writes ~8 KB, and each launch gives every workgroup one block (so launches of ~2048 workgroups follow
// each other; within one long launch the workgroups drift apart and reads and writes interleave at the memory). This
// kernel is shaped for that: 16 coordinates per lane (a team of 8 lanes per vector at D = 128, the whole wave at
// D = 1024), two passes per wave (16 or 2 vectors), no output staging (a store instruction writes, for each vector
// of a pass, the contiguous bytes its team holds: 128 bytes at D = 128, 1 KB at D = 1024), at most 64 VGPRs and a
// few KB of LDS; the host issues the call as launches of one block per workgroup.
#ifndef PITCH_STREAM_PASSES
#define PITCH_STREAM_PASSES 2  // vectors per wave of the streaming decoder = passes x 8
#endif
#ifndef PITCH_STREAM_NT
#define PITCH_STREAM_NT 1  // the streaming decoder writes with non-temporal stores
#endif
constexpr int kStreamE = 16;     // coordinates per lane: teams of 8 lanes at D = 128, 64 at D = 1024
constexpr int kStreamPasses = PITCH_STREAM_PASSES;
constexpr int kStreamWaves = 8;  // waves per SIMD the kernel is built for (64 VGPRs)

template <int D, int B, bool POLAR>
__global__ __launch_bounds__(kBlock, kStreamWaves) void vec_decode_stream(VecArgs p) {
  using G = Geom<D, kStreamE>;
  using TB = DecTab<B, POLAR, G::W>;
  static_assert((G::T == 8 || G::T == 64) && G::W == 4, "full 128-byte lines per team and chunk index");
  constexpr int NW = (D * B + 31) / 32;
  constexpr int CB = G::W * B;            // bits of codes per chunk (<= 32)
  constexpr int P = kStreamPasses;
  constexpr int VW = G::V * P;            // vectors per wave
  constexpr int WORDS = VW * NW;          // their code words, contiguous
  constexpr int NPL = (WORDS + 63) / 64;  // code words each lane loads
  __shared__ __attribute__((aligned(16))) float s_tab[TB::FLOATS];
  __shared__ uint32_t s_codes[kBlock / 64][WORDS];
  __shared__ float s_scale[kBlock / 64][VW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = lane & (G::T - 1), vw = lane / G::T;
  // this wave's VW vectors; a wave past the end takes the call's last VW vectors (the same bytes to the same places
  // as the wave that owns them), or the whole call when it has fewer
  const uint64_t nominal = ((uint64_t)blockIdx.x * (kBlock / 64) + wave) * VW;
  const uint64_t wb = p.count >= (uint64_t)VW ? (nominal < p.count - VW ? nominal : p.count - VW) : 0;
  // table source values and the sign word first, then the coalesced code and scale loads; waiting for the former
  // leaves the latter in flight (loads complete in order)
  const auto tab_src = load_dec_table<D, B, POLAR>();
  // the lane's 16 sign bits: one word per lane for teams of up to 32 lanes, two lanes per word for 64
  // (fill_stream_flips)
  const uint32_t fbits = G::T <= 32 ? p.lane_flips[t] : (p.lane_flips[t >> 1] >> (16 * (t & 1))) & 0xFFFFu;
  __builtin_amdgcn_sched_barrier(0);
  uint32_t w[NPL];
  {
    const uint32_t* cw = p.codes_in + wb * NW;
    const uint64_t last = p.count * NW - 1 - wb * NW;  // only binding in a call of fewer than VW vectors
#pragma unroll
    for (int m = 0; m < NPL; ++m) {
      const uint64_t i = (uint64_t)(lane + 64 * m < WORDS ? lane + 64 * m : WORDS - 1);
      w[m] = cw[i < last ? i : last];
    }
  }
  const uint64_t vs = wb + (uint64_t)(lane % VW);
  const float scale_l = p.scales_in[vs < p.count ? vs : p.count - 1];
  write_dec_table<D, B, POLAR>(tab_src, s_tab);
  asm volatile("" ::"v"(fbits));
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
  for (int m = 0; m < NPL; ++m) s_codes[wave][lane + 64 * m < WORDS ? lane + 64 * m : WORDS - 1] = w[m];
  if (lane < VW) s_scale[wave][lane] = scale_l;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // the butterflies at lane distances 4 and 8 as DPP operations (fwht_f32_lane_signed's WIDE) at D = 1024, where
  // they measured 2-6 % faster; at D = 128 the same form for distance 4 measured 8 % slower than a DPP move pair
  constexpr bool kWide = D >= 256;
  const uint32_t lane_sign = dpp_lane_sign_bit<D, kStreamE, kWide>(t);
  const uint64_t lastv = p.count - 1 - wb;
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const int lv0 = j * G::V + vw;
    const int lv = (uint64_t)lv0 < lastv ? lv0 : (int)lastv;  // past the end (a short call): the last vector
    const uint32_t* row = s_codes[wave] + lv * NW;
    float y[G::E];
#pragma unroll
    for (int k = 0; k < G::CH; ++k) {
      const int pos = CB * (k * G::T + t);
      const int wl = pos >> 5, wh = (pos & 31) + CB > 32 ? wl + 1 : wl;
      decode_chunk<D, B, POLAR>(__builtin_amdgcn_alignbit(row[wh], row[wl], (uint32_t)(pos & 31)), s_tab,
                                y + k * G::W);
    }
    fwht_f32_lane_signed<D, TB::PRE, kStreamE, kWide>(y, t);
    const float f = dec_scale<D>(s_scale[wave][lv], lane_sign);
    const uint64_t v = wb + (uint64_t)lv;
#pragma unroll
    for (int k = 0; k < G::CH; ++k) {
      float o[G::W];
#pragma unroll
      for (int r = 0; r < G::W; ++r) {
        const int e = k * G::W + r;
        o[r] = dec_out(y[e], f, ((fbits >> e) & 1u) << 31);
      }
      store_elems<0, G::W>(p.out, v * D + G::W * (k * G::T + t), o, PITCH_STREAM_NT);
    }
  }
}

// ----------------------------------------------------------------------------------------------------
// Lane-per-vector TurboQuant encoder, D in 8..128. A workgroup is one wave; it stages V = 64 / T vectors per
// iteration through LDS with coalesced 1 KB loads (16-bit inputs are widened to float32 at staging), after
// which each team of T lanes (T = 1 up to D = 32, D / 32 above) holds its vector as E = D / T contiguous
// float64 coordinates: coordinate c = t * E + e. The transform runs in registers plus DPP exchanges across
// the team, the rotation signs are applied at staging, codes are packed in registers and written back
// through LDS as contiguous wave stores.
template <int D, int IO>
struct Lpv {
  static constexpr int T = D <= PITCH_LPV_EMAX ? 1 : D / PITCH_LPV_EMAX;  // lanes per vector
  static constexpr int E = D / T;
  static constexpr int V = 64 / T;        // vectors per wave iteration
  static constexpr int HALF = E + 4;      // staged floats per team lane (padding spreads lanes over the banks)
  static constexpr int STRIDE = T * HALF; // staged floats per vector
  static constexpr int K = Io<IO>::kPerChunk;  // input elements per 16-byte chunk
  static constexpr int QPV = D / K;       // 16-byte chunks per vector
  static constexpr int QPL = V * QPV / 64;  // 16-byte chunks each lane loads per iteration
  static_assert(E % K == 0 && (V * QPV) % 64 == 0, "a chunk stays inside one team lane's coordinates");
};

// Coalesced load of the wave's block of V vectors as raw 16-byte chunks (vectors past the end re-read the
// last one).
template <int D, int IO>
__device__ __forceinline__ void lpv_fetch(const void* in, uint64_t base, uint64_t count, int lane,
                                         u32x4 (&pf)[Lpv<D, IO>::QPL]) {
  using Lp = Lpv<D, IO>;
  constexpr int EB = Io<IO>::kBytes;
  const char* bytes = (const char*)in;
  if (base + Lp::V <= count) {
    // whole block: the wave reads V * D contiguous elements, 1 KB per instruction
    const char* blk = bytes + base * D * EB + 16 * lane;
#pragma unroll
    for (int i = 0; i < Lp::QPL; ++i) pf[i] = *(const u32x4*)(blk + 1024 * i);
  } else {
#pragma unroll
    for (int i = 0; i < Lp::QPL; ++i) {
      const int q = lane + 64 * i;
      const int vq = q / Lp::QPV, pq = q % Lp::QPV;
      const uint64_t vg = base + vq < count ? base + vq : count - 1;
      pf[i] = *(const u32x4*)(bytes + (vg * D + Lp::K * pq) * EB);
    }
  }
}

// The K elements of a raw 16-byte chunk as float32 (exact).
template <int IO>
__device__ __forceinline__ void chunk_floats(const u32x4& w, float (&f)[Io<IO>::kPerChunk]) {
  if constexpr (IO == 0) {
    f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y); f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
  } else {
    widen2<IO>(w.x, f[0], f[1]); widen2<IO>(w.y, f[2], f[3]);
    widen2<IO>(w.z, f[4], f[5]); widen2<IO>(w.w, f[6], f[7]);
  }
}

#ifndef PITCH_ENC_FAIR
#define PITCH_ENC_FAIR 1  // persistent encoders raise a wave's issue priority with its share of blocks still to do
#endif
// A SIMD issues from its oldest wave first. With a fixed share of blocks per wave, the first-dispatched workgroups
// of a persistent encoder ran ahead and finished early, and the rest ended the call with fewer resident waves to
// hide their latency (a config-2 encode: every wave started within 0.4 us and ended between 11 and 23 us). In a
// persistent launch (on) each wave therefore sets its priority (s_setprio 0 .. 3) from the fraction of its blocks
// still to do, so the waves behind are issued first and a SIMD's waves finish together. An oversubscribed launch,
// where the hardware starts new workgroups as others finish, keeps the default priority (measured 1-1.5 % slower
// with it). Both arguments are wave-uniform.
struct FairPriority {
  bool on;
  float inv;      // 4 / the wave's blocks
  uint32_t left;  // blocks still to do
  // rem: vectors from the wave's first block to the end of its segment; stride: vectors between its blocks. The
  // block count ceil(rem / stride) is taken in float32 (to within one, which a priority level does not need better),
  // and only in a persistent launch: on a call's critical path a 64-bit division costs more than the priority saves.
  __device__ FairPriority(bool on_, uint64_t rem, uint64_t stride) : on(PITCH_ENC_FAIR && on_), inv(0.f), left(0u) {
    if (on) {
      const float q = __builtin_ceilf((float)rem * __builtin_amdgcn_rcpf((float)stride));
      const float blocks = __builtin_fminf(__builtin_fmaxf(1.f, q), 16777216.f);  // a count uint32_t holds exactly
      inv = 4.f * __builtin_amdgcn_rcpf(blocks);
      left = (uint32_t)blocks;
    }
  }
  // before each block
  __device__ __forceinline__ void next() {
    if (on) {
      const uint32_t level = __builtin_amdgcn_readfirstlane(min(3u, (uint32_t)((float)left * inv)));
      if (level >= 3) __builtin_amdgcn_s_setprio(3);
      else if (level == 2) __builtin_amdgcn_s_setprio(2);
      else if (level == 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
      left = left > 0 ? left - 1 : 0;
    }
  }
};

template <int D, int B, int IO, bool KBIAS>
__device__ __forceinline__ void lpv_run(const VecArgs& p, const EncSeg sg, uint64_t block, uint64_t nblocks) {
  using Lp = Lpv<D, IO>;
  constexpr int K = Lp::K;
  constexpr int E = Lp::E, T = Lp::T, V = Lp::V;
  constexpr int L = 1 << B;
  constexpr int NW = (D * B + 31) / 32;   // code words per vector
  constexpr int NWL = (E * B + 31) / 32;  // code words per lane (E * B is a multiple of 32 when T > 1)
  using Q = TqQuant<D, B>;
  static_assert(T == 1 || (E * B) % 32 == 0, "lanes of a team own whole code words");
  __shared__ __attribute__((aligned(16))) float s_in[V * Lp::STRIDE];
  __shared__ __attribute__((aligned(16))) uint32_t s_codes[V * NW];
  __shared__ typename Q::Smem s_q;

  const int lane = threadIdx.x;
  const int t = lane & (T - 1);
  const int vw = lane / T;
#if PITCH_ENC_PREFETCH
  // software pipeline: the next block's loads are in flight while this block is computed; the first block's
  // loads are issued before the table set-up so the two latencies overlap
  u32x4 pf[Lp::QPL];
  if (block * V < sg.count) lpv_fetch<D, IO>(sg.in, block * V, sg.count, lane, pf);
#endif
  Q::load(s_q, lane, 64);
  // Every 16-byte chunk this lane stages holds coordinates K * pq .. K * pq + K - 1 with pq = lane % QPV (64 is
  // a multiple of QPV), so the rotation signs are applied at staging with K fixed sign-bit masks.
  static_assert(64 % Lp::QPV == 0, "staged chunk positions are fixed per lane");
  uint32_t smask[K];
#pragma unroll
  for (int r = 0; r < K; ++r)
    smask[r] = sign_is_negative(p.seed, (uint32_t)(K * (lane % Lp::QPV) + r)) ? 0x80000000u : 0u;
  __syncthreads();
  FairPriority fair(p.fair != 0, block * V < sg.count ? sg.count - block * V : 0, nblocks * V);
  for (uint64_t base = block * V; base < sg.count; base += nblocks * V) {
    fair.next();
    // stage the wave's block of V vectors in LDS with coalesced loads
    {
#if !PITCH_ENC_PREFETCH
      u32x4 pf[Lp::QPL];
      lpv_fetch<D, IO>(sg.in, base, sg.count, lane, pf);
#endif
#pragma unroll
      for (int i = 0; i < Lp::QPL; ++i) {
        const int q = lane + 64 * i;
        const int vq = q / Lp::QPV, pq = q % Lp::QPV;
        const int h = (K * pq) / E, pe = K * pq - h * E;
        float fv[K];
        chunk_floats<IO>(pf[i], fv);
        if constexpr (KBIAS) {  // key-bias removal: encode x - o (mechanism_eval.py:113-116)
          float o[K];
          key_bias_offset<D, K>(p, base + vq < sg.count ? base + vq : sg.count - 1, K * pq, o);
#pragma unroll
          for (int r = 0; r < K; ++r) fv[r] = fv[r] - o[r];
        }
#pragma unroll
        for (int r = 0; r < K; ++r) fv[r] = __uint_as_float(__float_as_uint(fv[r]) ^ smask[r]);
#pragma unroll
        for (int r = 0; r < K; r += 4)
          *(float4*)(s_in + vq * Lp::STRIDE + h * Lp::HALF + pe + r) = float4{fv[r], fv[r + 1], fv[r + 2], fv[r + 3]};
      }
#if PITCH_ENC_PREFETCH
      const uint64_t nb = base + nblocks * V;
      if (nb < sg.count) lpv_fetch<D, IO>(sg.in, nb, sg.count, lane, pf);
#endif
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // this lane's E coordinates c = t * E + e, signs already applied (exact)
    double x[E];
#pragma unroll
    for (int k = 0; k < E / 4; ++k) {
      const float4 f = *(const float4*)(s_in + vw * Lp::STRIDE + t * Lp::HALF + 4 * k);
      x[4 * k] = (double)f.x;
      x[4 * k + 1] = (double)f.y;
      x[4 * k + 2] = (double)f.z;
      x[4 * k + 3] = (double)f.w;
    }

    // u = H(s * x) / (||x|| sqrt(d)) as in vec_encode (pitch_reference.py:96-98)
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < E; ++e) ss = __builtin_fma(x[e], x[e], ss);
    ss = team_reduce<T>(ss, [](double a, double b) { return a + b; });
    const double nrm = __builtin_sqrt(ss);
    const double us = (1.0 / (nrm > 0.0 ? nrm : 1.0)) * DimConst<D>::kInvSqrt;
    fwht_contig<E, T, double>(x, t);

    // code = #{edges < u} (pitch_reference.py:101), packed in registers (code of coordinate e at bit e * B)
    uint32_t w[NWL];
    Q::codes_packed(s_q, x, us, w);
#pragma unroll
    for (int i = 0; i < NWL; ++i) s_codes[vw * NW + t * NWL + i] = w[i];
    if (t == 0 && base + vw < sg.count) sg.scales_out[base + vw] = (float)nrm;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // write the wave's V * NW code words contiguously, in the widest chunks that stay inside one vector
    constexpr int CW = NW % 4 == 0 ? 4 : (NW % 2 == 0 ? 2 : 1);
    uint32_t* dst = sg.codes_out + base * NW;
#pragma unroll
    for (int i = 0; i < (V * NW / CW + 63) / 64; ++i) {
      const int q = lane + 64 * i;
      if (q < V * NW / CW && base + (q * CW) / NW < sg.count) {
        if constexpr (CW == 4) *(u32x4*)(dst + 4 * q) = *(const u32x4*)(s_codes + 4 * q);
        else if constexpr (CW == 2) *(u32x2*)(dst + 2 * q) = *(const u32x2*)(s_codes + 2 * q);
        else dst[q] = s_codes[q];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

template <int D, int B, int IO, bool KBIAS>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(PITCH_ENC_WAVES)))
void tq_encode_lpv(VecArgs p) {
  lpv_run<D, B, IO, KBIAS>(p, call_segment(p), blockIdx.x, gridDim.x);
}

template <int D, int B, int IO>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(PITCH_ENC_WAVES)))
void tq_encode_lpv_batch(VecBatchArgs pb) {
  const BatchSlot s = batch_slot(pb);
  lpv_run<D, B, IO, false>(pb.common, s.seg, s.block, s.blocks);
}

// ----------------------------------------------------------------------------------------------------
// Per-vector encoder (TurboQuant and PolarQuant) for float32 vectors at D = 64 and 128 with the transform's
// top stages applied at staging. A compute team of T lanes holds one vector, E = D / T contiguous coordinates per lane
// (c = t * E + e), so every stage left after staging runs inside a lane and each lane's codes are whole,
// contiguous code words (or, for E * B not a multiple of 32, words shared with one neighbour). The stages on
// the team bits (coordinate bits log2 E .. log2 D - 1) run while staging: staging lane p of a vector loads the
// T chunks at coordinates 4p + E * i (i < T), applies the rotation signs, widens to float64, applies those
// log2 T butterfly stages and writes the results to the LDS rows of the compute lanes that own them. The SL =
// E / 4 staging lanes of a vector read 4E contiguous bytes per load instruction, so the loads stay coalesced,
// and no cross-lane butterfly (two DPP moves and an add per float64 coordinate) is left.
template <int D, int T>
struct Hs {
  static constexpr int E = D / T;        // coordinates per compute lane
  static constexpr int V = 64 / T;       // vectors per wave iteration
  static constexpr int SL = E / 4;       // staging lanes per vector
  static constexpr int VPS = 64 / SL;    // vectors per load set (one load instruction per chunk i)
  static constexpr int NSET = V / VPS;   // load sets per wave iteration
  static constexpr int QPL = T * NSET;   // 16-byte chunks each lane loads per iteration
  // The sets are staged one at a time through LDS rows for VPS vectors: the compute lanes of set s read
  // their rows before set s + 1 is staged. Rows are padded so that the 8 lanes of each 128-byte access phase
  // hit distinct banks, for the staging writes (consecutive positions 4 pp, and vectors) and for the compute
  // reads (team lanes, and vectors): elements 16 apart are 36 banks apart when E > 16 (eoff), lane rows are
  // 8 banks apart (LS = 4 mod 16) and vectors 4 banks apart modulo 8 (VS = 2 mod 4).
  static constexpr int LS = E > 16 ? E + 4 : E + 4;  // float64 per compute lane row (E = 16: 20, E = 32: 36)
  static constexpr int VS = T * LS + 2;              // float64 per vector
  static constexpr int ROWS = VPS * VS;              // float64 of LDS rows per wave
  static constexpr int WAVES = kBlock / 64;  // independent waves per workgroup (they share the bucket table)
  __host__ __device__ static constexpr int eoff(int e) { return E > 16 ? e + 2 * (e / 16) : e; }
  static_assert(T >= 2 && E % 4 == 0 && 64 % SL == 0 && V % VPS == 0, "staging geometry");
  static_assert(eoff(E - 1) < LS && (2 * LS) % 32 == 8 && VS % 4 == 2, "row padding");
};

#ifndef PITCH_HS_T64
#define PITCH_HS_T64 4  // team lanes per vector of the staged-stage TurboQuant encoder at D = 64 (2 or 4)
#endif

template <int D>
constexpr int hs_team() { return D == 64 ? PITCH_HS_T64 : 4; }

#ifndef PITCH_HS_NT
#define PITCH_HS_NT 1  // the staged-stage encoder streams its input in and its codes and scales out non-temporally
#endif

#ifndef PITCH_HS_NTL
#define PITCH_HS_NTL PITCH_HS_NT  // the staged-stage encoder's loads alone
#endif

// One 16-byte load of the staged-stage encoder's input. Non-temporal: an encode reads each input byte once,
// and keeping the stream out of the caches lets the few writes interleave with it better (measured: +5 % at
// the same instruction count).
__device__ __forceinline__ u32x4 hs_load(const float* p) {
  if constexpr (PITCH_HS_NTL) return __builtin_nontemporal_load((const u32x4*)p);
  else return *(const u32x4*)p;
}
// The 16-bit form: the four elements of a staging lane's chunk are 8 bytes.
__device__ __forceinline__ u32x2 hs_load(const uint16_t* p) {
  if constexpr (PITCH_HS_NTL) return __builtin_nontemporal_load((const u32x2*)p);
  else return *(const u32x2*)p;
}
// What a staging lane loads per chunk of four elements: 16 bytes of float32, 8 of float16 / bfloat16.
template <int IO>
using HsChunk = typename std::conditional<IO == 0, u32x4, u32x2>::type;
template <int IO>
using HsElem = typename std::conditional<IO == 0, float, uint16_t>::type;
// The chunk's four elements as float32 (16-bit ones widened exactly).
template <int IO>
__device__ __forceinline__ void hs_chunk_floats(const HsChunk<IO>& c, float (&f)[4]) {
  if constexpr (IO == 0) {
    f[0] = __uint_as_float(c.x); f[1] = __uint_as_float(c.y); f[2] = __uint_as_float(c.z); f[3] = __uint_as_float(c.w);
  } else {
    widen2<IO>(c.x, f[0], f[1]);
    widen2<IO>(c.y, f[2], f[3]);
  }
}

// Coalesced loads of a wave's block of V vectors: set s, chunk i of lane l is vector base + s * VPS + l / SL
// at coordinates 4 * (l % SL) + E * i (vectors past the end re-read the last one).
template <int D, int T, int IO>
__device__ __forceinline__ void hs_fetch(const HsElem<IO>* in, uint64_t base, uint64_t count, int lane,
                                        HsChunk<IO> (&pf)[Hs<D, T>::QPL]) {
  using H = Hs<D, T>;
  const int vl = lane / H::SL, pp = lane % H::SL;
  if (base + H::V <= count) {
    const HsElem<IO>* blk = in + (base + vl) * D + 4 * pp;
#pragma unroll
    for (int s = 0; s < H::NSET; ++s)
#pragma unroll
      for (int i = 0; i < T; ++i) pf[s * T + i] = hs_load(blk + (uint64_t)s * H::VPS * D + H::E * i);
  } else {
#pragma unroll
    for (int s = 0; s < H::NSET; ++s) {
      const uint64_t v = base + s * H::VPS + vl;
      const HsElem<IO>* row = in + (v < count ? v : count - 1) * D + 4 * pp;
#pragma unroll
      for (int i = 0; i < T; ++i) pf[s * T + i] = hs_load(row + H::E * i);
    }
  }
}

// sqrt(n2) rounded as the library's float64 sqrt and h ~ 1 / (2 sqrt(n2)) to about an ulp, for n2 > 0 in
// the range of sums of squares of finite float32 values (2^-300 .. 2^264), which needs none of the range
// scaling of the general routine: the reciprocal square root estimate refined by one Goldschmidt step,
// two Newton corrections of the root and one more step of h.
__device__ __forceinline__ double sqrt_and_half_rsqrt(double n2, double& h) {
  const double y = __builtin_amdgcn_rsq(n2);
  double g = n2 * y;
  h = 0.5 * y;
  double r = __builtin_fma(-h, g, 0.5);
  g = __builtin_fma(g, r, g);
  h = __builtin_fma(h, r, h);
  double dd = __builtin_fma(-g, g, n2);
  g = __builtin_fma(dd, h, g);
  dd = __builtin_fma(-g, g, n2);
  g = __builtin_fma(dd, h, g);
  r = __builtin_fma(-h, g, 0.5);
  h = __builtin_fma(h, r, h);
  return g;
}

#ifndef PITCH_HS_PFD64
#define PITCH_HS_PFD64 1  // blocks of loads the staged-stage encoder keeps in flight per wave at D = 64 (1, 2)
#endif
#ifndef PITCH_HS_PFD128
#define PITCH_HS_PFD128 1  // the same at D = 128
#endif
// (one block where the key-bias variant's or the shared-word packing's extra registers leave no room for two)
template <int D, int B, bool KBIAS>
constexpr int hs_pfd() { return (KBIAS || B == 5 || B == 7) ? 1 : (D == 64 ? PITCH_HS_PFD64 : PITCH_HS_PFD128); }

// f, negated in the lanes whose bit of the wave-uniform mask is set: one v_cndmask with a negated operand and
// the mask as its lane-select scalar register pair.
__device__ __forceinline__ float neg_lanes(float f, uint64_t lanes) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, -%1, %2" : "=v"(r) : "v"(f), "s"(lanes));
  return r;
}

// Lane masks of the rotation signs for the staged-stage encoder (host side): bit l of mask i * 4 + k is set when
// coordinate 4 (l % SL) + E i + k, the one lane l stages as element k of chunk i, has sign -1.
static_assert(offsetof(VecArgs, lane_flips) % 8 == 0, "lane_flips is read as 64-bit lane masks");
template <int D, int T>
void fill_hs_flips(uint32_t seed, uint32_t* out) {
  using H = Hs<D, T>;
  static_assert(T * 4 * 2 <= 32, "masks fit in VecArgs::lane_flips");
  thread_local uint32_t cached_seed = 0;
  thread_local bool have = false;
  thread_local uint32_t cached[32];
  if (!have || cached_seed != seed) {
    for (int j = 0; j < 32; ++j) cached[j] = 0u;
    for (int i = 0; i < T; ++i)
      for (int k = 0; k < 4; ++k)
        for (int l = 0; l < 64; ++l)
          if (sign_is_negative(seed, (uint32_t)(4 * (l % H::SL) + H::E * i + k)))
            cached[2 * (i * 4 + k) + (l >> 5)] |= 1u << (l & 31);
    cached_seed = seed;
    have = true;
  }
  for (int j = 0; j < 32; ++j) out[j] = cached[j];
}

// Staging of one block (see Hs), one load set at a time: signs, float64, the butterfly stages on the team
// bits, the LDS rows of the set's compute lanes, which then read their coordinates into x. neg[i * 4 + k] is
// the lane mask of the sign of element k of chunk i (fill_hs_flips).
template <int D, int T, bool KBIAS, int IO>
__device__ __forceinline__ void hs_stage(const VecArgs& p, uint64_t count, const HsChunk<IO> (&pf)[Hs<D, T>::QPL],
                                         uint64_t base, int lane, const uint64_t* neg, double* sx,
                                         double (&x)[Hs<D, T>::E]) {
  using H = Hs<D, T>;
  constexpr int E = H::E;
  const int pp = lane % H::SL, vs = lane / H::SL;
  const int t = lane % T, vw = lane / T;
#pragma unroll
  for (int s = 0; s < H::NSET; ++s) {
    double y[T][4];
#pragma unroll
    for (int i = 0; i < T; ++i) {
      float f[4];
      hs_chunk_floats<IO>(pf[s * T + i], f);
      if constexpr (KBIAS) {  // key-bias removal: encode x - o (mechanism_eval.py:113-116)
        float o[4];
        const uint64_t v = base + s * H::VPS + vs;
        key_bias_offset<D, 4>(p, v < count ? v : count - 1, 4 * pp + E * i, o);
#pragma unroll
        for (int k = 0; k < 4; ++k) f[k] = f[k] - o[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) y[i][k] = (double)neg_lanes(f[k], neg[i * 4 + k]);
    }
#pragma unroll
    for (int h = 1; h < T; h <<= 1)
#pragma unroll
      for (int i = 0; i < T; ++i)
        if (!(i & h))
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const double a = y[i][k], b = y[i | h][k];
            y[i][k] = a + b;
            y[i | h][k] = a - b;
          }
#pragma unroll
    for (int i = 0; i < T; ++i) {
      double* row = sx + vs * H::VS + i * H::LS + H::eoff(4 * pp);
      *(double2*)row = double2{y[i][0], y[i][1]};
      *(double2*)(row + 2) = double2{y[i][2], y[i][3]};
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (H::NSET == 1 || vw / H::VPS == s) {
      const double* row = sx + (vw % H::VPS) * H::VS + t * H::LS;
#pragma unroll
      for (int k = 0; k < E / 2; ++k) {
        const double2 v2 = *(const double2*)(row + H::eoff(2 * k));
        x[2 * k] = v2.x;
        x[2 * k + 1] = v2.y;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// PolarQuant codes of the lane's E contiguous coordinates after the in-lane stages (pitch_reference.py:109-121):
// pairs (y_2p, y_2p+1) -> radius code floor(r / rmax * (2^B - 1) + 0.5) clipped and angle code
// floor(theta / 2 pi * 2^B + 0.5) mod 2^B, rmax = the largest radius of the vector (team-reduced). The codes
// depend only on the directions and on the radii relative to rmax, which the division by sqrt(d) of rotate()
// leaves unchanged (up to float64 rounding, far inside the near-boundary band): the pairs come from the
// unnormalised transform and only rmax is scaled. Each pair is decided in float32 on the unscaled pair (the
// angle is scale-invariant; the radius is multiplied by (2^B - 1) / rmax): the radius behind
// polar_radius_guard, the angle by sector_code at B <= 5 and by angle_sectors behind kPolarGuard above. A pair
// that fails a guard, and every pair of a vector whose rmax lies outside [1e-15, 1e18], is decided afterwards by
// the float64 path in the reference's order, in one block per lane that the waves enter only when one of their
// lanes has such a pair. The range keeps the float32 squared radius a^2 + c^2 exact to its rounding: near a
// radius boundary (r >= rmax / (2 (2^B - 1))) a subnormal square's absolute rounding error (2^-150 each) moves t
// by at most (2^B - 1)^2 2^-149 / rmax^2, under 1e-10 for rmax >= 1e-15 (for rmax near 1e-25 the squares
// underflow and every radius would read 0), and r <= rmax <= 1e18 keeps r^2 <= 1e36 below float32's largest
// value.
template <int B, int NWL>
__device__ __forceinline__ void put_code(uint32_t (&w)[NWL], int pos, uint32_t cd, bool clear) {
  const int wi = pos >> 5, sh = pos & 31;
  constexpr uint32_t M = (1u << B) - 1u;
  if (clear) w[wi] &= ~(M << sh);
  w[wi] |= cd << sh;
  if (sh + B > 32) {
    if (clear) w[wi + 1] &= ~(M >> (32 - sh));
    w[wi + 1] |= cd >> (32 - sh);
  }
}

template <int D, int T, int B, int NWL>
__device__ __forceinline__ float hs_polar_codes(double (&x)[D / T], uint32_t (&w)[NWL], lds_u8_t* otab) {
  constexpr int E = D / T, NP = E / 2, L = 1 << B;
  constexpr bool kSectors = B <= 5;
  constexpr float kRg = polar_radius_guard<B>();
  fwht_contig<E, 1, double>(x, 0);
  double m = 0.0;
#pragma unroll
  for (int q = 0; q < NP; ++q) m = __builtin_fmax(__builtin_fma(x[2 * q], x[2 * q], x[2 * q + 1] * x[2 * q + 1]), m);
  m = team_reduce<T>(m, [](double a, double b) { return __builtin_fmax(a, b); });
  const double rmax = __builtin_sqrt(m);  // = the largest radius: sqrt is monotone
  const double safe = rmax > 0.0 ? rmax : 1.0;
  const bool inrange = rmax >= 1e-15 && rmax <= 1e18;
  const float sr = (float)(double(L - 1) / safe);
#pragma unroll
  for (int i = 0; i < NWL; ++i) w[i] = 0u;
  bool okq[NP];
  bool all = true;
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const float af = (float)x[2 * q], cf = (float)x[2 * q + 1];
    const float rf = __builtin_amdgcn_sqrtf(__builtin_fmaf(af, af, cf * cf));
    // rf <= rmax up to rounding, so t_r < 2^B - 1/2 + 1e-5 and its floor needs no clip
    bool ok = inrange;
    const uint32_t cr = guarded_code_shifted(__builtin_fmaf(rf, sr, 0.5f - kRg), kRg, ok);
    uint32_t ca;
    if constexpr (kSectors) {
      if constexpr (PITCH_POLAR_OCT_TAB) ca = sector_code_tab<B>(cf, af, ok, otab);
      else ca = sector_code<B>(cf, af, ok);
    } else {  // a pair at the origin gives a NaN angle (0 * 1/0), which fails the guard
      ca = guarded_code_shifted(angle_sectors<B>(cf, af) + (0.5f - kPolarGuard), kPolarGuard, ok) &
           (uint32_t)(L - 1);
    }
    okq[q] = ok;
    all = all && ok;
    put_code<B>(w, 2 * q * B, cr, false);
    put_code<B>(w, (2 * q + 1) * B, ca, false);
  }
  if (!all) {  // rare
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      if (!okq[q]) {
        const double a = x[2 * q], c = x[2 * q + 1];
        const uint2 cc = polar_codes_exact<B>(a, c, __builtin_fma(a, a, c * c), safe);
        put_code<B>(w, 2 * q * B, cc.x, true);
        put_code<B>(w, (2 * q + 1) * B, cc.y, true);
      }
    }
  }
  return (float)div_sqrt_d<D>(rmax);
}

// Compute phase of one block: the in-lane stages, the quantisation (TurboQuant: norm and bucket table;
// PolarQuant: hs_polar_codes) and the stores.
template <int D, int T, int B, bool POLAR>
__device__ __forceinline__ void hs_compute(const EncSeg& sg, const typename TqLut8<D, B>::Smem& sq, uint64_t base,
                                           int lane, double* sx, double (&x)[Hs<D, T>::E]) {
  using H = Hs<D, T>;
  using Q = TqLut8<D, B>;
  constexpr int E = H::E, V = H::V;
  constexpr int NW = (D * B + 31) / 32;            // code words per vector
  constexpr bool kWhole = (E * B) % 32 == 0;       // each lane owns whole code words
  constexpr int NWL = (E * B + 31) / 32;           // code words a lane packs (first one shared when !kWhole)
  static_assert(kWhole || (T == 4 && E == 16 && B % 2 == 1), "shared code words: D = 64, T = 4, odd B");
  const int t = lane % T, vw = lane / T;
  uint32_t w[NWL];
  float nrm;
  if constexpr (POLAR) {
    nrm = hs_polar_codes<D, T, B, NWL>(x, w, (lds_u8_t*)sq.tab);
  } else {
    // ||x||^2 = sum of squares after the team-bit stages / T (each stage doubles it exactly)
    double ss[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int e = 0; e < E; ++e) ss[e & 3] = __builtin_fma(x[e], x[e], ss[e & 3]);
    double n2 = (ss[0] + ss[1]) + (ss[2] + ss[3]);
    n2 = team_reduce<T>(n2, [](double a, double b) { return a + b; }) * (1.0 / T);
    fwht_contig<E, 1, double>(x, 0);
    double h;
    const double g = sqrt_and_half_rsqrt(n2, h);
    const bool zero = !(n2 > 0.0);
    nrm = zero ? 0.f : (float)g;
    // u = H(s * x) / (||x|| sqrt(d)) (pitch_reference.py:96-98); a zero vector is divided by 1
    const double us = zero ? DimConst<D>::kInvSqrt : (2.0 * h) * DimConst<D>::kInvSqrt;
    Q::template codes_packed<(E > 16 ? 8 : PITCH_QBATCH)>(sq, x, us, lane, w);
  }
  // Every store is unconditional, so the compiler can count the vector-memory operations of an iteration and
  // wait for the next block's loads without waiting for these stores (gfx9 counts loads and stores together,
  // in order). A vector past the end was loaded from the last vector (hs_fetch), so its codes and scale equal
  // the last vector's and are written to that vector's place: the same bytes to the same address.
  const uint64_t vst = base + vw < sg.count ? base + vw : sg.count - 1;
  // the T lanes of a team write the same scale; cached (a wave writes 64 bytes of scales, half a line, which L2
  // merges with the next wave's)
  sg.scales_out[vst] = nrm;
  if constexpr (kWhole) {
    // lane (vw, t) owns words t * NWL .. of its vector: the wave's stores are one contiguous run
    if constexpr (PITCH_HS_NT) store_words_nt(sg.codes_out + vst * NW + t * NWL, w);
    else store_words(sg.codes_out + vst * NW + t * NWL, w);
  } else {
    // E * B = 16 B bits per lane: odd lanes start half-way into a word. Shift their bits up by 16, then
    // the even lane of each pair takes the odd lane's first (shared) word into its last one.
    if (t & 1) {
#pragma unroll
      for (int j = NWL - 1; j > 0; --j) w[j] = __builtin_amdgcn_alignbit(w[j], w[j - 1], 16);
      w[0] <<= 16;
    }
    const uint32_t shared = xchg_u32<1>(w[0]);
    if (!(t & 1)) w[NWL - 1] |= shared;
    __builtin_amdgcn_wave_barrier();
    uint32_t* sc = (uint32_t*)sx;  // the LDS rows were read into registers while staging
    static_assert(V * NW <= 2 * H::ROWS, "codes fit in the rows");
    const int w0 = (E * B * t) / 32;
#pragma unroll
    for (int j = 0; j < NWL; ++j)
      if (j > 0 || !(t & 1)) sc[vw * NW + w0 + j] = w[j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // V * NW / CW chunks of CW words, contiguous; lanes past the last chunk repeat it, and chunks of vectors
    // past the end go to the last vector's place (their words are the same)
    constexpr int CW = NW % 4 == 0 ? 4 : (NW % 2 == 0 ? 2 : 1);
    constexpr int NCH = V * NW / CW, CPV = NW / CW;
#pragma unroll
    for (int i = 0; i < (NCH + 63) / 64; ++i) {
      const int q = min(lane + 64 * i, NCH - 1);
      const int vq = q / CPV;
      const uint64_t vd = base + vq < sg.count ? base + vq : sg.count - 1;
      uint32_t* dst = sg.codes_out + vd * NW + CW * (q - vq * CPV);
      if constexpr (CW == 4) store_v((u32x4*)dst, *(const u32x4*)(sc + 4 * q), PITCH_HS_NT);
      else if constexpr (CW == 2) store_v((u32x2*)dst, *(const u32x2*)(sc + 2 * q), PITCH_HS_NT);
      else store_v(dst, sc[q], PITCH_HS_NT);
    }
  }
}

// Waves per SIMD the staged-stage encoder's registers must allow (its LDS allows 3; the key-bias variant's
// extra registers would spill at 3).
#ifndef PITCH_HS_WAVES64
#define PITCH_HS_WAVES64 3
#endif
#ifndef PITCH_HS_WAVES128
#define PITCH_HS_WAVES128 3
#endif
#ifndef PITCH_HS_WAVES_POLAR
#define PITCH_HS_WAVES_POLAR 3  // PolarQuant: 3 (a few spills, in the float64 fallback call only; LDS allows 3)
#endif
template <int D, bool POLAR, bool KBIAS>
constexpr int hs_waves() {
  return POLAR ? PITCH_HS_WAVES_POLAR : (KBIAS ? 2 : (D == 64 ? PITCH_HS_WAVES64 : PITCH_HS_WAVES128));
}

template <int D, int B, bool POLAR, bool KBIAS, int IO>
__device__ __forceinline__ void hs_run(const VecArgs& p, const EncSeg sg, uint64_t block, uint64_t nblocks) {
  constexpr int T = hs_team<D>();
  using H = Hs<D, T>;
  constexpr int E = H::E, V = H::V;
  using Q = TqLut8<D, B>;
  __shared__ __attribute__((aligned(16))) double s_x[H::WAVES][H::ROWS];
  __shared__ __attribute__((aligned(16))) typename Q::Smem s_q;  // (unused by PolarQuant)
  static_assert(sizeof(s_x) == hs_rows_bytes(D), "staging rows as the table copies assume");
  static_assert(!POLAR || sizeof(s_q) >= (size_t)OctTab<B>::N, "the octant table fits the bucket table's space");

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const HsElem<IO>* in = (const HsElem<IO>*)sg.in;
  const uint64_t stride = nblocks * H::WAVES * V;
  uint64_t base = (block * H::WAVES + wave) * V;
  // Software pipeline with PFD blocks of loads in flight. The loop is rotated so that each block's loads are
  // waited for in straight-line code after exactly the stores of the block before (two or so operations):
  // an iteration issues the loads of block k + PFD, computes and stores block k, then stages block k + 1.
  // The waves' first loads are issued after the table set-up, so no other load is pending at that point (issued
  // before it, with the table's loads queued behind them, small calls measured 2-13 % slower).
  constexpr int PFD = hs_pfd<D, B, KBIAS>();
  static_assert(PFD == 1 || PFD == 2, "prefetch depth");
  if constexpr (!POLAR) Q::template load<64 * H::WAVES>(s_q, threadIdx.x);
  else if constexpr (B <= 5 && PITCH_POLAR_OCT_TAB) octant_table_build<B>((uint8_t*)s_q.tab, threadIdx.x, 64 * H::WAVES);
  const uint64_t* neg = (const uint64_t*)p.lane_flips;  // fill_hs_flips; kernel arguments, read as scalars
  __syncthreads();
  if (base >= sg.count) return;
  HsChunk<IO> pfa[H::QPL];
  HsChunk<IO> pfb[PFD > 1 ? H::QPL : 1];
  // every fetch is unconditional, like the stores: a block past the end re-reads the last vector (a cache hit)
  hs_fetch<D, T, IO>(in, base, sg.count, lane, pfa);
  if constexpr (PFD > 1) hs_fetch<D, T, IO>(in, base + stride, sg.count, lane, pfb);
  double* sx = s_x[wave];
  double x[E];
  FairPriority fair(p.fair != 0, sg.count - base, stride);
  hs_stage<D, T, KBIAS, IO>(p, sg.count, pfa, base, lane, neg, sx, x);
  auto step = [&](HsChunk<IO> (&refill)[H::QPL], HsChunk<IO> (&next)[H::QPL]) {
    fair.next();
    hs_fetch<D, T, IO>(in, base + (uint64_t)PFD * stride, sg.count, lane, refill);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out before the compute, not interleaved into it
    hs_compute<D, T, B, POLAR>(sg, s_q, base, lane, sx, x);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the next block's staging waits for its loads: keep all of it after the compute
    __builtin_amdgcn_sched_barrier(0);
    base += stride;
    hs_stage<D, T, KBIAS, IO>(p, sg.count, next, base, lane, neg, sx, x);  // past the end: staged, never computed
  };
  if constexpr (PFD > 1) {
    while (true) {
      step(pfa, pfb);
      if (base >= sg.count) break;
      step(pfb, pfa);
      if (base >= sg.count) break;
    }
  } else {
    while (base < sg.count) step(pfa, pfa);
  }
}

template <int D, int B, bool POLAR, bool KBIAS, int IO>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(hs_waves<D, POLAR, KBIAS>())))
void vec_encode_hs(VecArgs p) {
  hs_run<D, B, POLAR, KBIAS, IO>(p, call_segment(p), blockIdx.x, gridDim.x);
}

template <int D, int B, bool POLAR, int IO>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(hs_waves<D, POLAR, false>())))
void vec_encode_hs_batch(VecBatchArgs pb) {
  const BatchSlot s = batch_slot(pb);
  hs_run<D, B, POLAR, false, IO>(pb.common, s.seg, s.block, s.blocks);
}

// ----------------------------------------------------------------------------------------------------
// LDS-transposed encoder for float32 vectors at D = 256, 512 and 1024 (both methods). A vector is held by a
// team of T = D / 32 lanes, twice over:
// - staging: team lane p loads the D / 32 chunks of CW = 1024 / D consecutive floats at coordinates
//   CW p + 32 j (j = 0 .. T - 1; each load instruction reads 128 contiguous bytes of every vector), applies the
//   rotation signs (one v_cndmask with a lane mask each), widens to float64 and runs the butterfly stages on
//   coordinate bits 5 and above in registers (they select the chunk j);
// - compute: after an exchange through LDS (row j of a vector = coordinates 32 j .. 32 j + 31), team lane q holds
//   the 32 contiguous coordinates 32 q + e and runs the stages on bits 0 .. 4 in registers.
// No butterfly crosses lanes (the team encoder at these sizes exchanges float64 values between lanes at 5 of
// the 10 stages, two moves and an fma per coordinate and stage), and each lane packs its 32 codes into B whole
// words. The LDS exchange takes two passes, each for half of every vector's rows (COLS: half of every row's
// columns, which keeps fewer registers live), so a wave needs 8.5 (9) KB of LDS. Measured at d = 256 .. 1024:
// TurboQuant is 1-2 % faster with the row split at 2 waves per SIMD (its column split holds 140 VGPRs, 3 waves,
// and gains nothing from them), PolarQuant 2-4 % faster with the column split at 3 waves.
template <int D, bool COLS>
struct Lt {
  static constexpr int T = D / 32;          // team lanes per vector
  static constexpr int V = 64 / T;          // vectors per wave iteration
  static constexpr int CW = 1024 / D;       // consecutive floats per staged chunk
  static constexpr int NJ = 32 / CW;        // chunks per staging lane (= T)
  // float64 per LDS row of a pass: 32 (16 columns) and 2 of padding, so rows are 16 bytes apart modulo 128 and
  // 8 lanes reading 16 bytes each hit distinct banks
  static constexpr int RS = COLS ? 18 : 34;
  static constexpr int HR = COLS ? T : T / 2;  // rows of a vector staged per pass
  static constexpr int ROWS = V * HR * RS;  // float64 of LDS per wave
  static constexpr int WAVES = kBlock / 64;
  static_assert(D >= 256 && D <= 1024 && NJ == T && HR >= 1, "geometry");
};

// Lane masks of the rotation signs (host side): bit b of word j * CW + r is set when coordinate
// CW (b % T) + r + 32 j, the one lane b (and lane b + 32) stages as element r of chunk j, has sign -1.
template <int D>
void fill_lt_flips(uint32_t seed, uint32_t* out) {
  using L = Lt<D, false>;
  static_assert(L::NJ * L::CW == 32, "one mask word per staged coordinate of a lane");
  thread_local uint32_t cached_seed = 0;
  thread_local bool have = false;
  thread_local uint32_t cached[32];
  if (!have || cached_seed != seed) {
    for (int j = 0; j < L::NJ; ++j)
      for (int r = 0; r < L::CW; ++r) {
        uint32_t m = 0u;
        for (int b = 0; b < 32; ++b)
          if (sign_is_negative(seed, (uint32_t)(L::CW * (b % L::T) + r + 32 * j))) m |= 1u << b;
        cached[j * L::CW + r] = m;
      }
    cached_seed = seed;
    have = true;
  }
  for (int j = 0; j < 32; ++j) out[j] = cached[j];
}

// Non-temporal loads of the input and stores of the codes (each measured 1-2 % faster than the cached form).
#ifndef PITCH_LT_NTL
#define PITCH_LT_NTL 1
#endif
#ifndef PITCH_LT_NTS
#define PITCH_LT_NTS 1
#endif
// Loads of a wave's block of V vectors (vectors past the end re-read the last one).
template <int D>
__device__ __forceinline__ void lt_fetch(const float* in, uint64_t base, uint64_t count, int lane, uint32_t (&pf)[32]) {
  using L = Lt<D, false>;
  const uint64_t v = base + lane / L::T;
  const float* row = in + (v < count ? v : count - 1) * D + L::CW * (lane % L::T);
#pragma unroll
  for (int j = 0; j < L::NJ; ++j) {
    if constexpr (L::CW == 4) {
      const u32x4 c = PITCH_LT_NTL ? __builtin_nontemporal_load((const u32x4*)(row + 32 * j)) : *(const u32x4*)(row + 32 * j);
      pf[4 * j] = c.x, pf[4 * j + 1] = c.y, pf[4 * j + 2] = c.z, pf[4 * j + 3] = c.w;
    } else if constexpr (L::CW == 2) {
      const u32x2 c = PITCH_LT_NTL ? __builtin_nontemporal_load((const u32x2*)(row + 32 * j)) : *(const u32x2*)(row + 32 * j);
      pf[2 * j] = c.x, pf[2 * j + 1] = c.y;
    } else {
      pf[j] = PITCH_LT_NTL ? __builtin_nontemporal_load((const uint32_t*)(row + 32 * j)) : *(const uint32_t*)(row + 32 * j);
    }
  }
}

// Staging of one block (see Lt): signs, float64, the stages on coordinate bits 5 and above, then two passes
// through the wave's LDS rows, each for half of every vector's rows, after which lane q of a vector holds its
// coordinates 32 q .. 32 q + 31 in x.
template <int D, bool COLS>
__device__ __forceinline__ void lt_stage(const uint32_t* neg, const uint32_t (&pf)[32], int lane, double* sx,
                                         double (&x)[32]) {
  using L = Lt<D, COLS>;
  constexpr int CW = L::CW, NJ = L::NJ, HR = L::HR;
  double y[NJ][CW];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < CW; ++r) {
      const uint32_t m = neg[j * CW + r];
      y[j][r] = (double)neg_lanes(__uint_as_float(pf[j * CW + r]), (uint64_t)m | ((uint64_t)m << 32));
    }
#pragma unroll
  for (int h = 1; h < NJ; h <<= 1)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (!(j & h))
#pragma unroll
        for (int r = 0; r < CW; ++r) {
          const double a = y[j][r], b = y[j | h][r];
          y[j][r] = a + b;
          y[j | h][r] = a - b;
        }
  const int tl = lane % L::T;
  double* vrows = sx + (lane / L::T) * HR * L::RS;
  if constexpr (COLS) {
    // pass s: the lanes whose columns CW tl .. CW tl + CW - 1 lie in half s write all their rows, then every
    // lane reads columns 16 s .. 16 s + 15 of its row
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if ((CW * tl) / 16 == s) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          double* dst = vrows + j * L::RS + CW * tl - 16 * s;
          if constexpr (CW == 4) {
            *(double2*)dst = double2{y[j][0], y[j][1]};
            *(double2*)(dst + 2) = double2{y[j][2], y[j][3]};
          } else if constexpr (CW == 2) {
            *(double2*)dst = double2{y[j][0], y[j][1]};
          } else {
            *dst = y[j][0];
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const double* src = vrows + tl * L::RS;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double2 v2 = *(const double2*)(src + 2 * k);
        x[16 * s + 2 * k] = v2.x;
        x[16 * s + 2 * k + 1] = v2.y;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int jj = 0; jj < HR; ++jj) {
      double* dst = vrows + jj * L::RS + CW * tl;
      if constexpr (CW == 4) {
        *(double2*)dst = double2{y[s * HR + jj][0], y[s * HR + jj][1]};
        *(double2*)(dst + 2) = double2{y[s * HR + jj][2], y[s * HR + jj][3]};
      } else if constexpr (CW == 2) {
        *(double2*)dst = double2{y[s * HR + jj][0], y[s * HR + jj][1]};
      } else {
        *dst = y[s * HR + jj][0];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (tl / HR == s) {
      const double* src = vrows + (tl - s * HR) * L::RS;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const double2 v2 = *(const double2*)(src + 2 * k);
        x[2 * k] = v2.x;
        x[2 * k + 1] = v2.y;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Compute phase of one block: the stages on bits 0 .. 4, the quantisation (TurboQuant: norm and bucket table;
// PolarQuant: hs_polar_codes) and the stores. As in the staged-stage encoder every store is unconditional: a
// vector past the end was loaded from the last vector, so its codes and scale are that vector's.
template <int D, int B, bool POLAR>
__device__ __forceinline__ void lt_compute(const EncSeg& sg, const typename TqLut8<D, B>::Smem& sq, uint64_t base,
                                           int lane, double (&x)[32]) {
  using L = Lt<D, false>;
  using Q = TqLut8<D, B>;
  constexpr int NW = D * B / 32;  // code words per vector; a lane's 32 codes are B of them
  const int tl = lane % L::T;
  uint32_t w[B];
  float nrm;
  if constexpr (POLAR) {
    nrm = hs_polar_codes<D, L::T, B, B>(x, w, (lds_u8_t*)sq.tab);
  } else {
    // ||x||^2 = sum of squares after the staging stages / T (each stage doubles it exactly)
    double ss[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int e = 0; e < 32; ++e) ss[e & 3] = __builtin_fma(x[e], x[e], ss[e & 3]);
    double n2 = (ss[0] + ss[1]) + (ss[2] + ss[3]);
    n2 = team_reduce<L::T>(n2, [](double a, double b) { return a + b; }) * (1.0 / L::T);
    fwht_contig<32, 1, double>(x, 0);
    double h;
    const double g = sqrt_and_half_rsqrt(n2, h);
    const bool zero = !(n2 > 0.0);
    nrm = zero ? 0.f : (float)g;
    // u = H(s * x) / (||x|| sqrt(d)) (pitch_reference.py:96-98); a zero vector is divided by 1
    const double us = zero ? DimConst<D>::kInvSqrt : (2.0 * h) * DimConst<D>::kInvSqrt;
    Q::template codes_packed<8>(sq, x, us, lane, w);
  }
  const uint64_t v = base + lane / L::T;
  const uint64_t vst = v < sg.count ? v : sg.count - 1;
  sg.scales_out[vst] = nrm;
  if constexpr (PITCH_LT_NTS) store_words_nt(sg.codes_out + vst * NW + tl * B, w);
  else store_words(sg.codes_out + vst * NW + tl * B, w);
}

// waves per SIMD the LDS-transposed encoder's registers must allow (PolarQuant: a few spills in the float64
// fallback only)
template <bool POLAR>
constexpr int lt_waves() { return POLAR ? 3 : 2; }

template <int D, int B, bool POLAR>
__device__ __forceinline__ void lt_run(const VecArgs& p, const EncSeg sg, uint64_t block, uint64_t nblocks) {
  using L = Lt<D, POLAR>;
  using Q = TqLut8<D, B>;
  __shared__ __attribute__((aligned(16))) double s_x[L::WAVES][L::ROWS];
  __shared__ __attribute__((aligned(16))) typename Q::Smem s_q;  // (unused by PolarQuant)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float* in = (const float*)sg.in;
  const uint64_t stride = nblocks * L::WAVES * L::V;
  uint64_t base = (block * L::WAVES + wave) * L::V;
  static_assert(!POLAR || sizeof(s_q) >= (size_t)OctTab<B>::N, "the octant table fits the bucket table's space");
  // Software pipeline as in the staged-stage encoder: an iteration issues the loads of block k + 1, computes and
  // stores block k, then stages block k + 1 (past the end: re-reads of the last vector, staged, never computed).
  if constexpr (!POLAR) Q::template load<kBlock>(s_q, threadIdx.x);
  else if constexpr (B <= 5 && PITCH_POLAR_OCT_TAB) octant_table_build<B>((uint8_t*)s_q.tab, threadIdx.x, kBlock);
  const uint32_t* neg = p.lane_flips;  // fill_lt_flips; kernel arguments, read as scalars
  __syncthreads();
  if (base >= sg.count) return;
  uint32_t pf[32];
  lt_fetch<D>(in, base, sg.count, lane, pf);
  double* sx = s_x[wave];
  double x[32];
  FairPriority fair(p.fair != 0, sg.count - base, stride);
  lt_stage<D, POLAR>(neg, pf, lane, sx, x);
  while (base < sg.count) {
    fair.next();
    lt_fetch<D>(in, base + stride, sg.count, lane, pf);
    __builtin_amdgcn_sched_barrier(0);
    lt_compute<D, B, POLAR>(sg, s_q, base, lane, x);
    __builtin_amdgcn_sched_barrier(0);
    base += stride;
    lt_stage<D, POLAR>(neg, pf, lane, sx, x);
  }
}

template <int D, int B, bool POLAR>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(lt_waves<POLAR>())))
void vec_encode_lt(VecArgs p) {
  lt_run<D, B, POLAR>(p, call_segment(p), blockIdx.x, gridDim.x);
}

template <int D, int B, bool POLAR>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(lt_waves<POLAR>())))
void vec_encode_lt_batch(VecBatchArgs pb) {
  const BatchSlot s = batch_slot(pb);
  lt_run<D, B, POLAR>(pb.common, s.seg, s.block, s.blocks);
}

#ifndef PITCH_LT_ENCODER
#define PITCH_LT_ENCODER 1  // 1: float32 encode at D = 256 .. 1024 uses vec_encode_lt
#endif

#ifndef PITCH_HS_ENCODER
#define PITCH_HS_ENCODER 1  // 1: float32 TurboQuant encode at D = 64 / 128 uses vec_encode_hs
#endif
#ifndef PITCH_HS_POLAR
#define PITCH_HS_POLAR 1  // 1: float32 PolarQuant encode at D = 64 / 128 uses vec_encode_hs
#endif
// float16 / bfloat16 vectors: the staged-stage encoder (8-byte chunk loads, widened at staging) runs PolarQuant at
// D = 64 and 128 (measured 18 -> 29 % of peak at D = 64, 17 -> 33 % at 128, against the team encoder) and
// TurboQuant at D = 128 (40 -> 43 %, against the lane-per-vector encoder); TurboQuant at D = 64 stays on the
// lane-per-vector encoder (within +-3 % either way).
#ifndef PITCH_HS_IO16
#define PITCH_HS_IO16 1
#endif

template <int D>
constexpr bool use_lpv_encoder() { return D >= 8 && D <= 128; }

// The encoder a call runs; a batched encode runs the same one for each of its segments.
enum class EncKind { kStaged, kTransposed, kLanePerVector, kTeam };
template <int D, bool POLAR, int IO, bool KBIAS>
constexpr EncKind enc_kind() {
  if ((IO == 0 || (PITCH_HS_IO16 && !KBIAS && (POLAR || D == 128))) && (POLAR ? PITCH_HS_POLAR : PITCH_HS_ENCODER) &&
      (D == 64 || D == 128))
    return EncKind::kStaged;
  if (IO == 0 && !KBIAS && PITCH_LT_ENCODER && D >= 256) return EncKind::kTransposed;
  if (!POLAR && use_lpv_encoder<D>()) return EncKind::kLanePerVector;
  return EncKind::kTeam;
}
// Vectors a workgroup of that encoder (without key bias) takes per round.
template <int D, bool POLAR, int IO>
constexpr uint32_t enc_vectors_per_block() {
  constexpr EncKind k = enc_kind<D, POLAR, IO, false>();
  if constexpr (k == EncKind::kStaged) return Hs<D, hs_team<D>()>::WAVES * Hs<D, hs_team<D>()>::V;
  else if constexpr (k == EncKind::kTransposed) return Lt<D, POLAR>::WAVES * Lt<D, POLAR>::V;
  else if constexpr (k == EncKind::kLanePerVector) return Lpv<D, IO>::V;
  else return Geom<D>::VPB;
}

template <int D, int B, bool POLAR, int IO, bool KBIAS>
hipError_t launch_one(bool encode, const VecArgs& args, hipStream_t s) {
  using G = Geom<D>;
  VecArgs a = args;
  constexpr EncKind kEnc = enc_kind<D, POLAR, IO, KBIAS>();
  if constexpr (kEnc == EncKind::kStaged) {
    if (encode) {
      using H = Hs<D, hs_team<D>()>;
      fill_hs_flips<D, hs_team<D>()>(a.seed, a.lane_flips);
      const uint64_t need = (a.count + H::WAVES * H::V - 1) / (H::WAVES * H::V);
      const void* k = (const void*)&vec_encode_hs<D, B, POLAR, KBIAS, IO>;
      const uint64_t grid = encode_grid(k, need, 64 * H::WAVES);
      a.fair = need > grid && grid == persistent_grid(k, need, 64 * H::WAVES) ? 1u : 0u;
      const uint64_t rounds = KBIAS ? 0 : slice_rounds(0);
      if (rounds && need > grid * rounds) {
        constexpr int NW = (D * B + 31) / 32;
        const uint64_t per = grid * rounds * H::WAVES * H::V;  // vectors per launch
        for (uint64_t v0 = 0; v0 < a.count; v0 += per) {
          VecArgs b = a;
          b.count = a.count - v0 < per ? a.count - v0 : per;
          b.in = (const char*)a.in + v0 * D * Io<IO>::kBytes;
          b.codes_out = a.codes_out + v0 * NW;
          b.scales_out = a.scales_out + v0;
          const uint64_t nb = (b.count + H::WAVES * H::V - 1) / (H::WAVES * H::V);
          hipLaunchKernelGGL((vec_encode_hs<D, B, POLAR, KBIAS, IO>), dim3((uint32_t)(nb < grid ? nb : grid)),
                             dim3(64 * H::WAVES), 0, s, b);
        }
        return hipGetLastError();
      }
      hipLaunchKernelGGL((vec_encode_hs<D, B, POLAR, KBIAS, IO>), dim3((uint32_t)grid), dim3(64 * H::WAVES), 0, s, a);
      return hipGetLastError();
    }
  }
  if constexpr (kEnc == EncKind::kTransposed) {
    if (encode) {
      using L = Lt<D, POLAR>;
      fill_lt_flips<D>(a.seed, a.lane_flips);
      const uint64_t need = (a.count + L::WAVES * L::V - 1) / (L::WAVES * L::V);
      const void* k = (const void*)&vec_encode_lt<D, B, POLAR>;
      // persistent at every size: the oversubscribed grid of encode_grid measured 3-4 % slower on the d = 1024
      // sweep (2^20 vectors, 43 rounds)
      const uint64_t grid = persistent_grid(k, need);
      a.fair = need > grid ? 1u : 0u;
      hipLaunchKernelGGL((vec_encode_lt<D, B, POLAR>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
      return hipGetLastError();
    }
  }
  if constexpr (kEnc == EncKind::kLanePerVector) {
    if (encode) {
      constexpr int V = Lpv<D, IO>::V;
      const uint64_t need = (a.count + V - 1) / V;
      const void* k = (const void*)&tq_encode_lpv<D, B, IO, KBIAS>;
      const uint64_t grid = persistent_grid(k, need, 64);
      a.fair = need > grid ? 1u : 0u;
      hipLaunchKernelGGL((tq_encode_lpv<D, B, IO, KBIAS>), dim3((uint32_t)grid), dim3(64), 0, s, a);
      return hipGetLastError();
    }
  }
  fill_lane_flips<D>(a.seed, a.lane_flips);
  const uint64_t need = (a.count + G::VPB - 1) / G::VPB;
  if (encode) {
    const void* k = (const void*)&vec_encode<D, B, POLAR, IO, KBIAS>;
    const uint64_t grid = persistent_grid(k, need);
    hipLaunchKernelGGL((vec_encode<D, B, POLAR, IO, KBIAS>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  } else {
    // float32 calls of at least 2^19 vectors at d = 1024 (2 GB of output): the streaming decoder. At d = 128 one
    // workgroup per block of vec_decode (below) measured as fast as the streaming decoder at 2^25 vectors (config
    // 5's value cache, 69.6-69.7 against 69.1-69.9 % of peak in interleaved repeats) and 2-7 points faster at
    // 2^22-2^24 (b = 3, 4, 8 and PolarQuant; b = 2 within 0.5), so d = 128 runs it at every size.
    if constexpr (D == 1024 && IO == 0 && !KBIAS) {
      if (a.count >= stream_decode_min_vectors()) {
        using GS = Geom<D, kStreamE>;
        constexpr uint64_t kVpb = (uint64_t)GS::V * kStreamPasses * (kBlock / 64);  // vectors per workgroup
        const void* ks = (const void*)&vec_decode_stream<D, B, POLAR>;
        const uint64_t blocks = (a.count + kVpb - 1) / kVpb;
        // capped one-launch grid (above), else one block per resident workgroup per launch (1.5x, 2x, 3x and 4x as
        // many measured 3-6 % slower)
        constexpr int kCap = B <= PITCH_STREAM_CAP_BITS ? PITCH_STREAM_WG_PER_CU : 0;
        const uint64_t grid = kCap > 0 ? blocks : persistent_grid(ks, blocks);
        const uint32_t lds = lds_cap_bytes(ks, kCap);
        VecArgs b = a;
        fill_stream_flips<D>(a.seed, b.lane_flips);
        for (uint64_t b0 = 0; b0 < blocks; b0 += grid) {
          const uint64_t nb = blocks - b0 < grid ? blocks - b0 : grid, v0 = b0 * kVpb;
          b.count = a.count - v0 < nb * kVpb ? a.count - v0 : nb * kVpb;
          b.codes_in = a.codes_in + v0 * ((D * B + 31) / 32);
          b.scales_in = a.scales_in + v0;
          b.out = (float*)a.out + v0 * D;
          hipLaunchKernelGGL((vec_decode_stream<D, B, POLAR>), dim3((uint32_t)nb), dim3(kBlock), lds, s, b);
        }
        return hipGetLastError();
      }
    }
    const void* k = (const void*)&vec_decode<D, B, POLAR, IO, KBIAS>;
    // float32 calls writing 64 MB or more run one workgroup per block (the hardware hands the blocks out as
    // workgroups finish) instead of a persistent grid. Interleaved repeats on one box, same bytes: config 4 (917,504
    // vectors at d = 128, 470 MB) 74 -> 84-90 % of peak, d = 64 at 0.4-1.3 GB 75-83 -> 87-90 %, d = 128 at 1-1.5 GB
    // 64-68 -> 72-73 %, d = 256 and 1024 +3-16 points, 67-200 MB +1-6 points; 100 MB at d = 64 equal.
    const uint64_t out_bytes = a.count * D * 4;
    const bool one_per_wg = IO == 0 && out_bytes >= PITCH_DEC_ONE_PER_WG_MIN && out_bytes < PITCH_DEC_ONE_PER_WG_MAX;
    const uint64_t grid = one_per_wg ? (need < 0x7FFFFFFFull ? need : 0x7FFFFFFFull)
                                     : persistent_grid(k, need, kBlock, true);
    const uint64_t rounds = (KBIAS || one_per_wg) ? 0 : slice_rounds(0);
    if (rounds && need > grid * rounds) {
      constexpr int NW = (D * B + 31) / 32;
      const uint64_t per = grid * rounds * G::VPB;  // vectors per launch
      for (uint64_t v0 = 0; v0 < a.count; v0 += per) {
        VecArgs b = a;
        b.count = a.count - v0 < per ? a.count - v0 : per;
        b.codes_in = a.codes_in + v0 * NW;
        b.scales_in = a.scales_in + v0;
        b.out = (char*)a.out + v0 * D * Io<IO>::kBytes;
        const uint64_t g = (b.count + G::VPB - 1) / G::VPB < grid ? (b.count + G::VPB - 1) / G::VPB : grid;
        hipLaunchKernelGGL((vec_decode<D, B, POLAR, IO, KBIAS>), dim3((uint32_t)g), dim3(kBlock), 0, s, b);
      }
    } else {
      hipLaunchKernelGGL((vec_decode<D, B, POLAR, IO, KBIAS>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
    }
  }
  return hipGetLastError();
}

// Key-bias removal is compiled for float32 vectors only (the entry points that take it are float32).
template <int D, int B, bool POLAR>
hipError_t launch_method(bool encode, const VecArgs& a, hipStream_t s) {
  if constexpr (PITCH_IO == 0) {
    if (a.kb_bias) return launch_one<D, B, POLAR, PITCH_IO, true>(encode, a, s);
  } else {
    if (a.kb_bias) return hipErrorInvalidValue;
  }
  return launch_one<D, B, POLAR, PITCH_IO, false>(encode, a, s);
}

template <int D, int B>
hipError_t launch_bits(bool encode, bool polar, const VecArgs& a, hipStream_t s) {
  return polar ? launch_method<D, B, true>(encode, a, s) : launch_method<D, B, false>(encode, a, s);
}

}  // namespace

#define PITCH_CAT2(a, b) a##b
#define PITCH_CAT(a, b) PITCH_CAT2(a, b)

namespace {
// Workgroups of a batch's segments (block_start): segment i needs need_i = ceil(count_i / vpb) blocks; grid_for(total)
// is the grid a single call of all the batch's blocks would run, and each segment gets ceil(need_i / r) workgroups,
// r being that grid's blocks per workgroup, so a long segment's workgroups loop over its blocks as a single call's
// do (and a table set-up per workgroup is paid as often), while short segments get one workgroup each.
template <typename Args, typename GridFor>
uint32_t assign_blocks(Args& a, uint64_t vpb, GridFor grid_for) {
  uint64_t total = 0;
  for (uint32_t j = 0; j < a.items; ++j) total += (a.count[j] + vpb - 1) / vpb;
  const uint64_t grid = grid_for(total);
  const uint64_t r = grid < total ? (total + grid - 1) / grid : 1;
  uint64_t blocks = 0;
  for (uint32_t j = 0; j < a.items; ++j) {
    a.block_start[j] = (uint32_t)blocks;
    blocks += ((a.count[j] + vpb - 1) / vpb + r - 1) / r;
  }
  a.block_start[a.items] = (uint32_t)blocks;
  return (uint32_t)blocks;
}

template <int D, int B, bool POLAR>
hipError_t launch_batch(VecBatchArgs a, hipStream_t s) {
  constexpr EncKind k = enc_kind<D, POLAR, PITCH_IO, false>();
  constexpr uint64_t vpb = enc_vectors_per_block<D, POLAR, PITCH_IO>();
  if constexpr (k == EncKind::kStaged) {
    const void* kp = (const void*)&vec_encode_hs_batch<D, B, POLAR, PITCH_IO>;
    bool fair = false;  // a persistent grid of more than one round
    const dim3 grid(assign_blocks(a, vpb, [&](uint64_t t) {
      const uint64_t g = encode_grid(kp, t, kBlock);
      fair = t > g && g == persistent_grid(kp, t, kBlock);
      return g;
    }));
    a.common.fair = fair ? 1u : 0u;
    fill_hs_flips<D, hs_team<D>()>(a.common.seed, a.common.lane_flips);
    hipLaunchKernelGGL((vec_encode_hs_batch<D, B, POLAR, PITCH_IO>), grid, dim3(kBlock), 0, s, a);
  } else if constexpr (k == EncKind::kTransposed) {
    const void* kp = (const void*)&vec_encode_lt_batch<D, B, POLAR>;
    bool fair = false;
    const dim3 grid(assign_blocks(a, vpb, [&](uint64_t t) {
      const uint64_t g = persistent_grid(kp, t);
      fair = t > g;
      return g;
    }));
    a.common.fair = fair ? 1u : 0u;
    fill_lt_flips<D>(a.common.seed, a.common.lane_flips);
    hipLaunchKernelGGL((vec_encode_lt_batch<D, B, POLAR>), grid, dim3(kBlock), 0, s, a);
  } else if constexpr (k == EncKind::kLanePerVector) {
    const void* kp = (const void*)&tq_encode_lpv_batch<D, B, PITCH_IO>;
    bool fair = false;
    const dim3 grid(assign_blocks(a, vpb, [&](uint64_t t) {
      const uint64_t g = persistent_grid(kp, t, 64);
      fair = t > g;
      return g;
    }));
    a.common.fair = fair ? 1u : 0u;
    hipLaunchKernelGGL((tq_encode_lpv_batch<D, B, PITCH_IO>), grid, dim3(64), 0, s, a);
  } else {
    const void* kp = (const void*)&vec_encode_batch<D, B, POLAR, PITCH_IO>;
    const dim3 grid(assign_blocks(a, vpb, [&](uint64_t t) { return persistent_grid(kp, t); }));
    fill_lane_flips<D>(a.common.seed, a.common.lane_flips);
    hipLaunchKernelGGL((vec_encode_batch<D, B, POLAR, PITCH_IO>), grid, dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}
template <int D, int B>
hipError_t launch_batch_bits(bool polar, const VecBatchArgs& a, hipStream_t s) {
  return polar ? launch_batch<D, B, true>(a, s) : launch_batch<D, B, false>(a, s);
}
// A batched decode gives every block of every segment its own workgroup (the config-4 shape, 28 segments of 32,768
// vectors at d = 128, measured 78-80 us against 89-90 us for a persistent grid over the same vectors).
template <int D, int B, bool POLAR>
hipError_t launch_dec_batch(DecBatchArgs a, hipStream_t s) {
  const uint32_t blocks = assign_blocks(a, Geom<D>::VPB, [](uint64_t t) { return t; });
  fill_lane_flips<D>(a.common.seed, a.common.lane_flips);
  hipLaunchKernelGGL((vec_decode_batch<D, B, POLAR, PITCH_IO>), dim3(blocks), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}
template <int D, int B>
hipError_t launch_dec_batch_bits(bool polar, const DecBatchArgs& a, hipStream_t s) {
  return polar ? launch_dec_batch<D, B, true>(a, s) : launch_dec_batch<D, B, false>(a, s);
}
}  // namespace

hipError_t PITCH_CAT(PITCH_CAT(PITCH_CAT(launch_vec_dec_batch_d, PITCH_DIM), _io), PITCH_IO)(bool polar, int bits,
                                                                                        const DecBatchArgs& a,
                                                                                        hipStream_t s) {
  switch (bits) {
    case 2: return launch_dec_batch_bits<PITCH_DIM, 2>(polar, a, s);
    case 3: return launch_dec_batch_bits<PITCH_DIM, 3>(polar, a, s);
    case 4: return launch_dec_batch_bits<PITCH_DIM, 4>(polar, a, s);
    case 5: return launch_dec_batch_bits<PITCH_DIM, 5>(polar, a, s);
    case 6: return launch_dec_batch_bits<PITCH_DIM, 6>(polar, a, s);
    case 7: return launch_dec_batch_bits<PITCH_DIM, 7>(polar, a, s);
    case 8: return launch_dec_batch_bits<PITCH_DIM, 8>(polar, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t PITCH_CAT(PITCH_CAT(PITCH_CAT(launch_vec_batch_d, PITCH_DIM), _io), PITCH_IO)(bool polar, int bits,
                                                                                    const VecBatchArgs& a,
                                                                                    hipStream_t s) {
  switch (bits) {
    case 2: return launch_batch_bits<PITCH_DIM, 2>(polar, a, s);
    case 3: return launch_batch_bits<PITCH_DIM, 3>(polar, a, s);
    case 4: return launch_batch_bits<PITCH_DIM, 4>(polar, a, s);
    case 5: return launch_batch_bits<PITCH_DIM, 5>(polar, a, s);
    case 6: return launch_batch_bits<PITCH_DIM, 6>(polar, a, s);
    case 7: return launch_batch_bits<PITCH_DIM, 7>(polar, a, s);
    case 8: return launch_batch_bits<PITCH_DIM, 8>(polar, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t PITCH_CAT(PITCH_CAT(PITCH_CAT(launch_vec_d, PITCH_DIM), _io), PITCH_IO)(bool encode, bool polar, int bits,
                                                                              const VecArgs& a, hipStream_t s) {
  switch (bits) {
    case 2: return launch_bits<PITCH_DIM, 2>(encode, polar, a, s);
    case 3: return launch_bits<PITCH_DIM, 3>(encode, polar, a, s);
    case 4: return launch_bits<PITCH_DIM, 4>(encode, polar, a, s);
    case 5: return launch_bits<PITCH_DIM, 5>(encode, polar, a, s);
    case 6: return launch_bits<PITCH_DIM, 6>(encode, polar, a, s);
    case 7: return launch_bits<PITCH_DIM, 7>(encode, polar, a, s);
    case 8: return launch_bits<PITCH_DIM, 8>(encode, polar, a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pitch
