// Device-side building blocks shared by the codec kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "pitch_launch.h"
#include "pitch_tables.inc"

namespace pitch {

constexpr int kBlock = 256;  // threads per workgroup: four wave64s

// ---------------------------------------------------------------------------------------------------
// compile-time loop
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

// ---------------------------------------------------------------------------------------------------
// Rotation signs. pcg_hash as reference/pitch_reference.py:11-15 (PITCHKernels.metal:26-31); the sign of
// coordinate i is +1 when pcg_hash(seed + i) is odd and -1 when it is even (pitch_reference.py:17-19).
__host__ __device__ __forceinline__ uint32_t pcg_hash(uint32_t v) {
  const uint32_t state = v * 747796405u + 2891336453u;
  const uint32_t word = ((state >> ((state >> 28u) + 4u)) ^ state) * 277803737u;
  return (word >> 22u) ^ word;
}
__host__ __device__ __forceinline__ bool sign_is_negative(uint32_t seed, uint32_t i) {
  return (pcg_hash(seed + i) & 1u) == 0u;
}

// ---------------------------------------------------------------------------------------------------
// Cross-lane exchange with the lane at (lane ^ MASK). Lanes 1 and 2 apart use DPP quad permutes, 4 apart a
// half-row mirror followed by a quad reverse (i -> 7-i -> (7-i)^3 = i^4), 8 apart a row rotate by 8;
// 16 and 32 apart go through ds_bpermute. Every lane of the wave must be active.
template <int MASK>
__device__ __forceinline__ uint32_t xchg_u32(uint32_t x) {
  if constexpr (MASK == 1) {
    return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);  // quad_perm:[1,0,3,2]
  } else if constexpr (MASK == 2) {
    return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);  // quad_perm:[2,3,0,1]
  } else if constexpr (MASK == 4) {
    const uint32_t y = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true);  // row_half_mirror
    return __builtin_amdgcn_mov_dpp(y, 0x1B, 0xF, 0xF, true);               // quad_perm:[3,2,1,0]
  } else if constexpr (MASK == 8) {
    return __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);  // row_ror:8
  } else {
    static_assert(MASK == 16 || MASK == 32, "lane distance");
    const int src = (int)((__lane_id() ^ MASK) << 2);
    return (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)x);
  }
}
template <int MASK>
__device__ __forceinline__ float xchg(float x) {
  return __uint_as_float(xchg_u32<MASK>(__float_as_uint(x)));
}
template <int MASK>
__device__ __forceinline__ double xchg(double x) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = xchg_u32<MASK>((uint32_t)u);
  const uint32_t hi = xchg_u32<MASK>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ float fma_t(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_t(double a, double b, double c) { return __builtin_fma(a, b, c); }

// ---------------------------------------------------------------------------------------------------
// Register layout of one vector of D coordinates spread over a team of T consecutive lanes.
// Coordinates are grouped into chunks of W (4, or 2 when D == 2); lane t of the team holds chunks
// j = k*T + t for k = 0 .. CH-1, so consecutive lanes read consecutive 16-byte chunks and every global
// access of a wave is contiguous per vector. Element e = k*W + r of a lane is coordinate
// c = W*(k*T + t) + r: bits [0, lgW) of c select r (in registers), bits [lgW, lgW+lgT) select the team lane
// (exchanged across lanes) and the remaining bits select k (in registers).
#ifndef PITCH_E64
#define PITCH_E64 16  // coordinates per lane at D = 64
#endif
#ifndef PITCH_E128
#define PITCH_E128 32  // coordinates per lane at D = 128
#endif

constexpr int default_lane_coords(int D) {
  return D <= 16 ? D : (D == 64 ? PITCH_E64 : (D == 128 ? PITCH_E128 : (D < 64 ? 16 : 32)));
}

// EE: coordinates per lane (default: the decoders' and team encoders' choice for D)
template <int D, int EE = default_lane_coords(D)>
struct Geom {
  static constexpr int W = D >= 4 ? 4 : D;
  static constexpr int E = EE;
  static constexpr int T = D / E;
  static constexpr int CH = E / W;
  static constexpr int V = 64 / T;                  // vectors per wave
  static constexpr int VPB = V * (kBlock / 64);     // vectors per workgroup iteration
  static constexpr int LGD = ilog2(D), LGW = ilog2(W), LGT = ilog2(T);
  static_assert(T * E == D && CH * W == E && T <= 64, "geometry");
  __host__ __device__ static constexpr int coord(int t, int e) { return W * ((e / W) * T + t) + (e % W); }
};

// In-place unnormalised Walsh-Hadamard transform of one vector held by a team, with the stages in the
// reference's order (bit 0 first; reference/pitch_reference.py:21-31) and each butterfly computing
// exactly a + b and a - b, so a float64 transform reproduces the reference bit for bit.
// Cross-lane butterfly: the low lane computes fma(mine, +1, partner) = a + b, the high lane
// fma(mine, -1, partner) = a - b.
// min / max with the hardware's semantics, as single instructions: for non-NaN operands the same as fminf /
// fmaxf, without the canonicalising v_max_f32 x, x that the compiler puts before fminf / fmaxf (and before a
// med3 against an infinity, which it turns into them) for operands not known to be canonical, such as loaded
// values or values exchanged between lanes.
__device__ __forceinline__ float fmin_hw(float a, float b) { float r; asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b)); return r; }
__device__ __forceinline__ float fmax_hw(float a, float b) { float r; asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b)); return r; }
__device__ __forceinline__ float fmin3_hw(float a, float b, float c) {
  float r;
  asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float fmax3_hw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// RN(1 / x) for a per-channel step: v_rcp_f32 and one Newton step. On gfx950 this equals the correctly rounded
// reciprocal for every normal x below 2^126 (checked exhaustively by pitch_selftest_reciprocal); steps of the
// per-channel codec are at most (65504 + 65504) / 3. An infinite step (a range end beyond float16) gives 0,
// the reciprocal of infinity; a NaN step gives NaN.
__device__ __forceinline__ float rcp_rn(float x) {
  const float y0 = __builtin_amdgcn_rcpf(x);
  const float y1 = __builtin_fmaf(__builtin_fmaf(-x, y0, 1.0f), y0, y0);
  return __builtin_isinf(x) ? 0.0f : y1;
}

// floor(x) converted to int32 in one instruction (exact: the floor of a float is an integer-valued float; NaN
// gives 0 and values beyond the int32 range saturate). The compiler does not form it from (int)floorf(x).
__device__ __forceinline__ int cvt_flr_i32(float x) {
  int r;
  asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

template <int D, typename F>
__device__ __forceinline__ void fwht(F (&v)[Geom<D>::E], int t) {
  using G = Geom<D>;
  static_for<0, G::LGD>([&](auto bit_c) {
    constexpr int bit = decltype(bit_c)::value;
    if constexpr (bit >= G::LGW && bit < G::LGW + G::LGT) {
      constexpr int lm = 1 << (bit - G::LGW);
      const F sg = (t & lm) ? F(-1) : F(1);
#pragma unroll
      for (int e = 0; e < G::E; ++e) v[e] = fma_t(v[e], sg, xchg<lm>(v[e]));
    } else {
      constexpr int m = bit < G::LGW ? (1 << bit) : (G::W << (bit - G::LGW - G::LGT));
#pragma unroll
      for (int e = 0; e < G::E; ++e) {
        if (!(e & m)) {
          const F a = v[e], b = v[e | m];
          v[e] = a + b;
          v[e | m] = a - b;
        }
      }
    }
  });
}

// ---------------------------------------------------------------------------------------------------
// Cross-lane butterflies as one instruction per element. v_fmac_f32 with a DPP quad permute on its first
// operand computes v = partner * sg + v: with sg = +1 on the low lane of a pair and -1 on the high lane, the
// low lane gets a + b and the high lane b - a = -(a - b), each with the single rounding of a + b or a - b.
// The compiler does not form this instruction from mov_dpp + fma, hence the inline assembly. A DPP read
// needs two wait states after a VALU write of its source register: the leading s_nop covers the block's
// inputs, the trailing one a compiler-emitted DPP read of its outputs.
#ifndef PITCH_DPP_FMAC
#define PITCH_DPP_FMAC 1
#endif
#define PITCH_FMAC_DPP(I, PERM) "v_fmac_f32_dpp %" #I ", %" #I ", %16 " PERM " row_mask:0xf bank_mask:0xf\n"
#define PITCH_FMAC_DPP16(PERM)                                                                              \
  "s_nop 1\n" PITCH_FMAC_DPP(0, PERM) PITCH_FMAC_DPP(1, PERM) PITCH_FMAC_DPP(2, PERM) PITCH_FMAC_DPP(3, PERM) \
      PITCH_FMAC_DPP(4, PERM) PITCH_FMAC_DPP(5, PERM) PITCH_FMAC_DPP(6, PERM) PITCH_FMAC_DPP(7, PERM)          \
          PITCH_FMAC_DPP(8, PERM) PITCH_FMAC_DPP(9, PERM) PITCH_FMAC_DPP(10, PERM) PITCH_FMAC_DPP(11, PERM)   \
              PITCH_FMAC_DPP(12, PERM) PITCH_FMAC_DPP(13, PERM) PITCH_FMAC_DPP(14, PERM)                      \
                  PITCH_FMAC_DPP(15, PERM) "s_nop 1\n"

// LM = 8 pairs lane i with i ^ 8 through row_ror:8 (a rotation by half a row).
template <int LM, int O, int E>
__device__ __forceinline__ void fmac_dpp16(float (&v)[E], float sg) {
  static_assert((LM == 1 || LM == 2 || LM == 8) && O + 16 <= E, "DPP partners over 16 elements");
#define PITCH_FMAC_DPP_OPS                                                                                  \
  : "+v"(v[O]), "+v"(v[O + 1]), "+v"(v[O + 2]), "+v"(v[O + 3]), "+v"(v[O + 4]), "+v"(v[O + 5]),             \
    "+v"(v[O + 6]), "+v"(v[O + 7]), "+v"(v[O + 8]), "+v"(v[O + 9]), "+v"(v[O + 10]), "+v"(v[O + 11]),       \
    "+v"(v[O + 12]), "+v"(v[O + 13]), "+v"(v[O + 14]), "+v"(v[O + 15])                                      \
  : "v"(sg)
  if constexpr (LM == 1)
    asm(PITCH_FMAC_DPP16("quad_perm:[1,0,3,2]") PITCH_FMAC_DPP_OPS);
  else if constexpr (LM == 2)
    asm(PITCH_FMAC_DPP16("quad_perm:[2,3,0,1]") PITCH_FMAC_DPP_OPS);
  else
    asm(PITCH_FMAC_DPP16("row_ror:8") PITCH_FMAC_DPP_OPS);
#undef PITCH_FMAC_DPP_OPS
}

// The butterfly at lane distance 4 in two DPP operations per element, without a separate move: lanes 0-3 of each
// 8 (DPP banks 0 and 2) add the partner read through row_shl:4, lanes 4-7 (banks 1 and 3) take partner - own
// through row_shr:4 (each operation writes only its banks; both read the inputs, so neither sees the other's
// result). Low lanes get a + b, high lanes a - b, with the signs of the plain butterfly. Eight elements per block,
// with the DPP read hazard covered as in fmac_dpp16.
#define PITCH_BFLY4(O, I)                                                                                       \
  "v_add_f32_dpp %" #O ", %" #I ", %" #I " row_shl:4 row_mask:0xf bank_mask:0x5\n"                               \
  "v_sub_f32_dpp %" #O ", %" #I ", %" #I " row_shr:4 row_mask:0xf bank_mask:0xa\n"
template <int O, int E>
__device__ __forceinline__ void bfly4_dpp8(float (&v)[E]) {
  static_assert(O + 8 <= E, "eight elements");
  float r[8];
  asm("s_nop 1\n" PITCH_BFLY4(0, 8) PITCH_BFLY4(1, 9) PITCH_BFLY4(2, 10) PITCH_BFLY4(3, 11) PITCH_BFLY4(4, 12)
          PITCH_BFLY4(5, 13) PITCH_BFLY4(6, 14) PITCH_BFLY4(7, 15) "s_nop 1"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(v[O]), "v"(v[O + 1]), "v"(v[O + 2]), "v"(v[O + 3]), "v"(v[O + 4]), "v"(v[O + 5]), "v"(v[O + 6]),
        "v"(v[O + 7]));
#pragma unroll
  for (int i = 0; i < 8; ++i) v[O + i] = r[i];
}
#undef PITCH_BFLY4

// Lanes of the team whose cross-lane stages fwht_f32_lane_signed runs as v_fmac_f32_dpp (distances 1 and 2,
// when E is a multiple of 16; with WIDE also 8). These come out negated on the high lane of each pair.
template <int D, int EE = default_lane_coords(D), bool WIDE = false>
__host__ __device__ constexpr int dpp_lane_bits() {
  return (PITCH_DPP_FMAC && Geom<D, EE>::E % 16 == 0) ? ((WIDE ? 11 : 3) & (Geom<D, EE>::T - 1)) : 0;
}
// Sign bit that lane t's results of fwht_f32_lane_signed carry: (-1)^popcount(t & dpp_lane_bits).
template <int D, int EE = default_lane_coords(D), bool WIDE = false>
__device__ __forceinline__ uint32_t dpp_lane_sign_bit(int t) {
  return (uint32_t)(__builtin_popcount((unsigned)(t & dpp_lane_bits<D, EE, WIDE>())) & 1) << 31;
}

// fwht<D, float> with the cross-lane stages at distances 1 and 2 done by fmac_dpp16. The high lane of each
// such pair comes out negated, and every later butterfly pairs lanes that carry the same sign (they differ
// only in higher lane bits or are the same lane), so the factor passes through unchanged: lane t's results
// equal the transform times (-1)^popcount(t & dpp_lane_bits<D>()), bit for bit up to that sign (b - a
// and -(a - b) round alike; only a zero may come out with the other sign). The first PRE stages (bits
// below PRE <= log2 W, inside a chunk) are taken as already applied by the caller.
// With WIDE, the stage at lane distance 8 is a v_fmac_f32_dpp too (row_ror:8), and the one at distance 4 is
// bfly4_dpp8 (two DPP operations per element, signs as the plain butterfly's).
template <int D, int PRE = 0, int EE = default_lane_coords(D), bool WIDE = false>
__device__ __forceinline__ void fwht_f32_lane_signed(float (&v)[EE], int t) {
  using G = Geom<D, EE>;
  static_assert(PRE >= 0 && PRE <= G::LGW, "pre-applied stages lie inside a chunk");
  static_for<PRE, G::LGD>([&](auto bit_c) {
    constexpr int bit = decltype(bit_c)::value;
    if constexpr (bit >= G::LGW && bit < G::LGW + G::LGT) {
      constexpr int lm = 1 << (bit - G::LGW);
      const float sg = (t & lm) ? -1.0f : 1.0f;
      if constexpr ((dpp_lane_bits<D, EE, WIDE>() & lm) != 0) {
        static_for<0, G::E / 16>([&](auto o_c) { fmac_dpp16<lm, 16 * decltype(o_c)::value>(v, sg); });
      } else if constexpr (WIDE && lm == 4 && PITCH_DPP_FMAC && G::E % 8 == 0) {
        static_for<0, G::E / 8>([&](auto o_c) { bfly4_dpp8<8 * decltype(o_c)::value>(v); });
      } else {
#pragma unroll
        for (int e = 0; e < G::E; ++e) v[e] = fma_t(v[e], sg, xchg<lm>(v[e]));
      }
    } else {
      constexpr int m = bit < G::LGW ? (1 << bit) : (G::W << (bit - G::LGW - G::LGT));
#pragma unroll
      for (int e = 0; e < G::E; ++e) {
        if (!(e & m)) {
          const float a = v[e], b = v[e | m];
          v[e] = a + b;
          v[e | m] = a - b;
        }
      }
    }
  });
}

// Unnormalised Walsh-Hadamard transform of E contiguous coordinates per lane across a team of T lanes:
// coordinate c = t * E + e; stages in the reference's order, bits >= log2 E cross lanes.
template <int E, int T, typename F>
__device__ __forceinline__ void fwht_contig(F (&v)[E], int t) {
  static_for<0, ilog2(E) + ilog2(T)>([&](auto bit_c) {
    constexpr int bit = decltype(bit_c)::value;
    if constexpr (bit < ilog2(E)) {
      constexpr int m = 1 << bit;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if (!(e & m)) {
          const F a = v[e], b = v[e | m];
          v[e] = a + b;
          v[e | m] = a - b;
        }
      }
    } else {
      constexpr int lm = 1 << (bit - ilog2(E));
      const F sg = (t & lm) ? F(-1) : F(1);
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = fma_t(v[e], sg, xchg<lm>(v[e]));
    }
  });
}

// Reduction over the team (all lanes end with the result).
template <int T, typename F, typename Op>
__device__ __forceinline__ F team_reduce(F x, Op op) {
  static_for<0, ilog2(T)>([&](auto s_c) {
    constexpr int lm = 1 << decltype(s_c)::value;
    x = op(x, xchg<lm>(x));
  });
  return x;
}

// ---------------------------------------------------------------------------------------------------
// Unaligned (4-byte aligned) vector memory types: gfx950 global memory serves dword-aligned multi-dword
// accesses, so offsets that are multiples of 4 bytes still use 8/12/16-byte instructions.
typedef float f32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));

// ---------------------------------------------------------------------------------------------------
// Element type of the uncompressed vectors: what encode reads and decode writes. IO = 0 float32, 1 float16,
// 2 bfloat16 (PITCH_IO_F32 / PITCH_IO_F16 / PITCH_IO_BF16 of the C ABI). 16-bit elements are widened to
// float32 exactly on load; float32 results are rounded to nearest even on store (v_cvt_pk_f16_f32 /
// v_cvt_pk_bf16_f32; a value beyond the 16-bit range becomes infinity, as any RNE conversion does).
template <int IO>
struct Io {
  static_assert(IO >= 0 && IO <= 2, "I/O element type");
  static constexpr int kBytes = IO == 0 ? 4 : 2;
  static constexpr int kPerChunk = 16 / kBytes;  // elements per 16-byte access
};

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// The two 16-bit elements of w (element 0 in the low half) as float32.
template <int IO>
__device__ __forceinline__ void widen2(uint32_t w, float& a, float& b) {
  if constexpr (IO == 1) {
    a = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
    b = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  } else {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xFFFF0000u);
  }
}

// (a, b) rounded to the 16-bit type and packed, a in the low half.
#ifndef PITCH_F16_PACKED_CVT
#define PITCH_F16_PACKED_CVT 1  // float16: one v_cvt_pk_f16_f32 per pair (0: two v_cvt_f16_f32)
#endif
template <int IO>
__device__ __forceinline__ uint32_t narrow2(float a, float b) {
  const f32x2 v{a, b};
  if constexpr (IO == 1) {
    if constexpr (PITCH_F16_PACKED_CVT) {
      return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    } else {
      const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)a), hi = __builtin_bit_cast(uint16_t, (_Float16)b);
      return lo | (hi << 16);
    }
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  }
}

template <int IO>
__device__ __forceinline__ float widen1(uint16_t h) {
  float a, b;
  widen2<IO>((uint32_t)h, a, b);
  return a;
}

// Loads elements [i, i + N) of an IO-typed array as float32 (N = 1, 2, 4 or 8; one access of N elements).
template <int IO, int N>
__device__ __forceinline__ void load_elems(const void* base, uint64_t i, float (&f)[N]) {
  if constexpr (IO == 0) {
    const float* p = (const float*)base + i;
    if constexpr (N == 8) {
      const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else if constexpr (N == 4) {
      const f32x4 a = *(const f32x4*)p;
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    } else if constexpr (N == 2) {
      const f32x2 a = *(const f32x2*)p;
      f[0] = a.x; f[1] = a.y;
    } else {
      f[0] = *p;
    }
  } else {
    const uint16_t* p = (const uint16_t*)base + i;
    if constexpr (N == 8) {
      const u32x4 w = *(const u32x4*)p;
      widen2<IO>(w.x, f[0], f[1]); widen2<IO>(w.y, f[2], f[3]);
      widen2<IO>(w.z, f[4], f[5]); widen2<IO>(w.w, f[6], f[7]);
    } else if constexpr (N == 4) {
      const u32x2 w = *(const u32x2*)p;
      widen2<IO>(w.x, f[0], f[1]); widen2<IO>(w.y, f[2], f[3]);
    } else if constexpr (N == 2) {
      widen2<IO>(*(const uint32_t*)p, f[0], f[1]);
    } else {
      f[0] = widen1<IO>(*p);
    }
  }
}

// load_elems of 4 elements with a non-temporal load (an input streamed through once).
template <int IO>
__device__ __forceinline__ void load4_nt(const void* base, uint64_t i, float (&f)[4]) {
  if constexpr (IO == 0) {
    const f32x4 a = __builtin_nontemporal_load((const f32x4*)((const float*)base + i));
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  } else {
    const u32x2 w = __builtin_nontemporal_load((const u32x2*)((const uint16_t*)base + i));
    widen2<IO>(w.x, f[0], f[1]);
    widen2<IO>(w.y, f[2], f[3]);
  }
}

// Stores f[0, N) at elements [i, i + N) of an IO-typed array in one access, non-temporal when NT.
template <typename V>
__device__ __forceinline__ void store_v(V* p, V v, bool nt) {
  if (nt) __builtin_nontemporal_store(v, p);
  else *p = v;
}
template <int IO, int N>
__device__ __forceinline__ void store_elems(void* base, uint64_t i, const float (&f)[N], bool nt) {
  if constexpr (IO == 0) {
    float* p = (float*)base + i;
    if constexpr (N == 8) {
      store_v((f32x4*)p, f32x4{f[0], f[1], f[2], f[3]}, nt);
      store_v((f32x4*)(p + 4), f32x4{f[4], f[5], f[6], f[7]}, nt);
    } else if constexpr (N == 4) {
      store_v((f32x4*)p, f32x4{f[0], f[1], f[2], f[3]}, nt);
    } else if constexpr (N == 2) {
      store_v((f32x2*)p, f32x2{f[0], f[1]}, nt);
    } else {
      store_v(p, f[0], nt);
    }
  } else {
    uint16_t* p = (uint16_t*)base + i;
    if constexpr (N == 8) {
      store_v((u32x4*)p, u32x4{narrow2<IO>(f[0], f[1]), narrow2<IO>(f[2], f[3]), narrow2<IO>(f[4], f[5]),
                               narrow2<IO>(f[6], f[7])}, nt);
    } else if constexpr (N == 4) {
      store_v((u32x2*)p, u32x2{narrow2<IO>(f[0], f[1]), narrow2<IO>(f[2], f[3])}, nt);
    } else if constexpr (N == 2) {
      store_v((uint32_t*)p, narrow2<IO>(f[0], f[1]), nt);
    } else {
      store_v(p, (uint16_t)(narrow2<IO>(f[0], 0.f) & 0xFFFFu), nt);
    }
  }
}

// store_words with non-temporal stores (streamed out, not kept in the caches).
template <int N>
__device__ __forceinline__ void store_words_nt(uint32_t* dst, const uint32_t (&w)[N]) {
  int i = 0;
#pragma unroll
  for (; i + 4 <= N; i += 4) __builtin_nontemporal_store(u32x4{w[i], w[i + 1], w[i + 2], w[i + 3]}, (u32x4*)(dst + i));
  if constexpr (N % 4 == 3) __builtin_nontemporal_store(u32x3{w[i], w[i + 1], w[i + 2]}, (u32x3*)(dst + i));
  if constexpr (N % 4 == 2) __builtin_nontemporal_store(u32x2{w[i], w[i + 1]}, (u32x2*)(dst + i));
  if constexpr (N % 4 == 1) __builtin_nontemporal_store(w[i], dst + i);
}

template <int N>
__device__ __forceinline__ void store_words(uint32_t* dst, const uint32_t (&w)[N]) {
  int i = 0;
#pragma unroll
  for (; i + 4 <= N; i += 4) *(u32x4*)(dst + i) = u32x4{w[i], w[i + 1], w[i + 2], w[i + 3]};
  if constexpr (N % 4 == 3) *(u32x3*)(dst + i) = u32x3{w[i], w[i + 1], w[i + 2]};
  if constexpr (N % 4 == 2) *(u32x2*)(dst + i) = u32x2{w[i], w[i + 1]};
  if constexpr (N % 4 == 1) dst[i] = w[i];
}

// Packs 32 codes given as bytes (bytes[i] holds code i < 2^B) into B little-endian words: code i at bits
// [i*B, i*B + B) (reference/pitch_reference.py:68-78).
template <int B>
__device__ __forceinline__ void pack32(const uint32_t (&bytes)[8], uint32_t (&w)[B]) {
#pragma unroll
  for (int k = 0; k < B; ++k) w[k] = 0u;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t c = (bytes[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    const int pos = i * B, wi = pos >> 5, sh = pos & 31;
    w[wi] |= c << sh;
    if (sh + B > 32) w[wi + 1] |= c >> (32 - sh);
  }
}

}  // namespace pitch
