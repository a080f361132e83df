// Per-vector TurboQuant and single-level PolarQuant encode/decode for one dimension (PITCH_DIM).
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
#include "pitch_device.h"

#ifndef PITCH_DIM
#error "compile with -DPITCH_DIM=<dim>"
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

constexpr double kTwoPi = 0x1.921fb54442d18p+2;  // 2 * np.pi
constexpr double kInvTwoPi = 1.0 / kTwoPi;

// y / sqrt(D) rounded as the reference's division (pitch_reference.py:33).
template <int D>
__device__ __forceinline__ double div_sqrt_d(double y) {
  using C = DimConst<D>;
  if constexpr (C::kPow4) return y * C::kInvSqrt;
  else return div_rn(y, C::kSqrt, C::kInvSqrt);
}

template <int W>
__device__ __forceinline__ void load_chunk(const float* src, float (&f)[W]) {
  if constexpr (W == 4) {
    const f32x4 q = *(const f32x4*)src;
    f[0] = q.x; f[1] = q.y; f[2] = q.z; f[3] = q.w;
  } else {
    const f32x2 q = *(const f32x2*)src;
    f[0] = q.x; f[1] = q.y;
  }
}

#ifndef PITCH_NT_STORE
#define PITCH_NT_STORE 1  // decoded vectors are streamed out with nontemporal stores (0: regular stores)
#endif

template <int W>
__device__ __forceinline__ void store_chunk(float* dst, const float (&f)[W]) {
  if constexpr (W == 4) {
    if (PITCH_NT_STORE) __builtin_nontemporal_store(f32x4{f[0], f[1], f[2], f[3]}, (f32x4*)dst);
    else *(f32x4*)dst = f32x4{f[0], f[1], f[2], f[3]};
  } else {
    if (PITCH_NT_STORE) __builtin_nontemporal_store(f32x2{f[0], f[1]}, (f32x2*)dst);
    else *(f32x2*)dst = f32x2{f[0], f[1]};
  }
}

// ----------------------------------------------------------------------------------------------------
template <int D, int B, bool POLAR>
__global__ __launch_bounds__(kBlock) void vec_encode(VecArgs p) {
  using G = Geom<D>;
  constexpr int L = 1 << B;
  constexpr int NW = (D * B + 31) / 32;  // 32-bit words of codes per vector
  constexpr bool kStage = D >= 32;       // codes are packed from LDS in groups of 32
  __shared__ double s_edge[POLAR ? 1 : L];
  __shared__ __attribute__((aligned(16))) uint32_t s_stage[kStage ? G::VPB * D / 4 : 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int t = lane & (G::T - 1);
  const int slot = (tid >> 6) * G::V + lane / G::T;

  if constexpr (!POLAR) {
    constexpr int off = pitch_codebook_offset(ilog2(D), B);
    for (int i = tid; i < L; i += kBlock) s_edge[i] = (double)pitch_edge_tab[off + i];
  }
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
    const bool valid = !TAIL || v < p.count;
    const float* src = p.in + (valid ? v : p.count - 1) * D;

    // load every chunk before converting (all loads in flight together), then apply the signs (exact)
    float f[G::E];
#pragma unroll
    for (int k = 0; k < G::CH; ++k) load_chunk<G::W>(src + G::W * (k * G::T + t), *(float(*)[G::W])(f + k * G::W));
    __builtin_amdgcn_sched_barrier(0);
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
      // code = number of edges strictly below u: searchsorted(edges, u, 'left') (pitch_reference.py:101)
#pragma unroll
      for (int e = 0; e < G::E; ++e) {
        const double u = x[e] * us;
        uint32_t cd = 0;
#pragma unroll
        for (int s = L / 2; s >= 1; s >>= 1) cd = (u > s_edge[cd + s - 1]) ? cd + s : cd;
        code[e] = cd;
      }
    } else {
      fwht<D, double>(x, t);
#pragma unroll
      for (int e = 0; e < G::E; ++e) x[e] = div_sqrt_d<D>(x[e]);
      // pairs (y_2p, y_2p+1) -> radius and angle (pitch_reference.py:111-121)
      constexpr int NP = G::E / 2;
      double rad[NP];
      double rmax = 0.0;
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        const double a = x[2 * q], c = x[2 * q + 1];
        rad[q] = __builtin_sqrt(__builtin_fma(a, a, c * c));
        rmax = rad[q] > rmax ? rad[q] : rmax;
      }
      rmax = team_reduce<G::T>(rmax, [](double a, double b) { return a > b ? a : b; });
      const double safe = rmax > 0.0 ? rmax : 1.0;
      const double inv = 1.0 / safe;
      constexpr double RL = double(L - 1), N = double(L);
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        double rq = __builtin_floor(div_rn(rad[q], safe, inv) * RL + 0.5);
        rq = rq < 0.0 ? 0.0 : (rq > RL ? RL : rq);
        code[2 * q] = (uint32_t)rq;
        double th = atan2(x[2 * q + 1], x[2 * q]);
        if (th < 0.0) th += kTwoPi;  // np.mod(theta, 2 pi) for theta in [-pi, 0)
        const double tq = __builtin_floor(div_rn(th, kTwoPi, kInvTwoPi) * N + 0.5);
        code[2 * q + 1] = (uint32_t)tq & (uint32_t)(L - 1);
      }
      scale = (float)rmax;
    }

    if constexpr (kStage) {
#pragma unroll
      for (int k = 0; k < G::CH; ++k) {
        const int c0 = G::W * (k * G::T + t);
        s_stage[(slot * D + c0) >> 2] = code[4 * k] | (code[4 * k + 1] << 8) | (code[4 * k + 2] << 16) |
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
      if (valid) store_words<NW>(p.codes_out + v * NW, w);
    }
    if (t == 0 && valid) p.scales_out[v] = scale;

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
          if (!TAIL || vv < p.count) {
            const uint4* q = (const uint4*)(s_stage + ((vs * D + 32 * gi) >> 2));
            const uint4 q0 = q[0], q1 = q[1];
            const uint32_t bytes[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            uint32_t w[B];
            pack32<B>(bytes, w);
            store_words<B>(p.codes_out + vv * NW + gi * B, w);
          }
        }
      }
      __syncthreads();
    }
  };
  for (uint64_t base = (uint64_t)blockIdx.x * G::VPB; base < p.count;
       base += (uint64_t)gridDim.x * G::VPB) {
    if (base + G::VPB <= p.count) body(base, std::false_type{});
    else body(base, std::true_type{});
  }
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
};

template <int D, int B, bool POLAR>
__device__ __forceinline__ void build_dec_table(float* s_tab) {
  using TB = DecTab<B, POLAR, Geom<D>::W>;
  constexpr int L = TB::L;
  if constexpr (POLAR) {
    constexpr int off = pitch_polar_offset(B);
    const float* rad = pitch_polar_radius_tab + off;
    const float* cs = pitch_polar_cos_tab + off;
    const float* sn = pitch_polar_sin_tab + off;
    if constexpr (TB::G == 2) {
      for (int i = threadIdx.x; i < TB::ENTRIES; i += kBlock) {
        const float r = rad[i & (L - 1)];
        s_tab[2 * i] = r * cs[i >> B];
        s_tab[2 * i + 1] = r * sn[i >> B];
      }
    } else {
      for (int i = threadIdx.x; i < L; i += kBlock) {
        s_tab[i] = rad[i];
        s_tab[L + i] = cs[i];
        s_tab[2 * L + i] = sn[i];
      }
    }
  } else {
    const float* cb = pitch_codebook_tab + pitch_codebook_offset(ilog2(D), B);
    if constexpr (TB::G == 4) {
      for (int i = threadIdx.x; i < 256; i += kBlock) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s_tab[4 * i + r] = cb[(i >> (2 * r)) & 3];
      }
    } else if constexpr (TB::G == 2) {
      for (int i = threadIdx.x; i < TB::ENTRIES; i += kBlock) {
        s_tab[2 * i] = cb[i & (L - 1)];
        s_tab[2 * i + 1] = cb[i >> B];
      }
    } else {
      for (int i = threadIdx.x; i < L; i += kBlock) s_tab[i] = cb[i];
    }
  }
}

// Unpacks the W codes of one chunk (bits [0, W*B) of `bits`) into W rotated-domain values.
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

#ifndef PITCH_DEC_WAVES
#define PITCH_DEC_WAVES 1  // minimum waves per SIMD requested for the decoders (caps their VGPRs)
#endif

template <int D, int B, bool POLAR>
__global__ __launch_bounds__(kBlock, PITCH_DEC_WAVES) void vec_decode(VecArgs p) {
  using G = Geom<D>;
  using TB = DecTab<B, POLAR, G::W>;
  constexpr int NW = (D * B + 31) / 32;
  constexpr int CB = G::W * B;  // bits of codes per chunk (<= 32)
  __shared__ __attribute__((aligned(16))) float s_tab[TB::FLOATS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int t = lane & (G::T - 1);
  const int slot = (tid >> 6) * G::V + lane / G::T;

  build_dec_table<D, B, POLAR>(s_tab);
  const uint32_t fbits = p.lane_flips[t];
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
  __syncthreads();

  // Software pipeline: the codes and scale of the next iteration are loaded before the current one is
  // transformed, so every wave keeps a batch of loads in flight while it computes. Loads are unconditional
  // (indices past the end are clamped to the last vector); only lanes holding a real vector store.
  struct Batch {
    uint32_t lo[G::CH], hi[G::CH];
    float scale;
  };
  auto fetch = [&](uint64_t base) {
    Batch b;
    const uint64_t v = base + slot;
    const uint64_t vl = v < p.count ? v : p.count - 1;
    b.scale = p.scales_in[vl];
    const uint32_t* cw = p.codes_in + vl * NW;
#pragma unroll
    for (int k = 0; k < G::CH; ++k) {
      b.lo[k] = cw[wlo[k]];
      b.hi[k] = cw[whi[k]];
    }
    return b;
  };
  auto body = [&](const Batch& b, uint64_t base, auto tail_c) {
    constexpr bool TAIL = decltype(tail_c)::value;
    const uint64_t v = base + slot;
    const bool valid = !TAIL || v < p.count;
    float y[G::E];
#pragma unroll
    for (int k = 0; k < G::CH; ++k)
      decode_chunk<D, B, POLAR>(__builtin_amdgcn_alignbit(b.hi[k], b.lo[k], wsh[k]), s_tab, y + k * G::W);

    fwht<D, float>(y, t);

    const float f = b.scale * DimConst<D>::kInvSqrtF;
    if (valid) {
      float* dst = p.out + v * D;
#pragma unroll
      for (int k = 0; k < G::CH; ++k) {
        float o[G::W];
#pragma unroll
        for (int r = 0; r < G::W; ++r)
          o[r] = __uint_as_float(__float_as_uint(y[k * G::W + r] * f) ^ flip[k * G::W + r]);
        store_chunk<G::W>(dst + G::W * (k * G::T + t), o);
      }
    }
  };
  const uint64_t stride = (uint64_t)gridDim.x * G::VPB;
  uint64_t base = (uint64_t)blockIdx.x * G::VPB;
  if (base >= p.count) return;  // uniform per workgroup; no barrier follows
  Batch cur = fetch(base);
  for (;;) {
    const uint64_t nbase = base + stride;
    const Batch nxt = fetch(nbase < p.count ? nbase : base);
    if (base + G::VPB <= p.count) body(cur, base, std::false_type{});
    else body(cur, base, std::true_type{});
    if (nbase >= p.count) break;
    cur = nxt;
    base = nbase;
  }
}

// Per-team-lane sign bits for the seed (cached per thread for the last seed).
template <int D>
void fill_lane_flips(uint32_t seed, uint32_t* out) {
  using G = Geom<D>;
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

template <int D, int B, bool POLAR>
hipError_t launch_one(bool encode, const VecArgs& args, hipStream_t s) {
  using G = Geom<D>;
  VecArgs a = args;
  fill_lane_flips<D>(a.seed, a.lane_flips);
  const uint64_t need = (a.count + G::VPB - 1) / G::VPB;
  if (encode) {
    const void* k = (const void*)&vec_encode<D, B, POLAR>;
    const uint64_t grid = persistent_grid(k, need);
    hipLaunchKernelGGL((vec_encode<D, B, POLAR>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  } else {
    const void* k = (const void*)&vec_decode<D, B, POLAR>;
    const uint64_t grid = persistent_grid(k, need);
    hipLaunchKernelGGL((vec_decode<D, B, POLAR>), dim3((uint32_t)grid), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

template <int D, int B>
hipError_t launch_bits(bool encode, bool polar, const VecArgs& a, hipStream_t s) {
  return polar ? launch_one<D, B, true>(encode, a, s) : launch_one<D, B, false>(encode, a, s);
}

}  // namespace

#define PITCH_CAT2(a, b) a##b
#define PITCH_CAT(a, b) PITCH_CAT2(a, b)

hipError_t PITCH_CAT(launch_vec_d, PITCH_DIM)(bool encode, bool polar, int bits, const VecArgs& a,
                                             hipStream_t s) {
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
