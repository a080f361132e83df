// Decode-phase attention over compressed K and V caches, without decompressing them (one dimension per
// object file: PITCH_DIM = 64 or 128).
//
// The reference evaluates attention on decoded caches: S = Q K^T * scale, log-softmax, P V
// (reference/attention_extra.py:70-74, attention_eval.py:31-33), and names decoding inside attention as its
// next step (README.md:96). For the per-vector codecs the decode is x = s (.) H(t[c]) * n / sqrt(d)
// (pitch_reference.py:104-107, 123-129): t is the method's value table (Lloyd-Max centroids, or radius fraction
// times (cos, sin) for PolarQuant pairs), n the stored scale, s the rotation signs and H the symmetric
// Walsh-Hadamard matrix. Hence
//   q . k_t       = n_t / sqrt(d) * sum_j (H (s_K (.) q))_j t[c_tj]     (the query is rotated once)
//   sum_t p_t v_t = s_V (.) H( sum_t p_t n_t t[c_t] ) / sqrt(d)          (one inverse rotation per query)
// so no token is transformed: per token and coordinate pair the kernels do one LDS table read and a few FMAs
// on the codes as stored. Kernels of one call (flash-decoding over chunks of a KV head's tokens):
//   attn_prep     q'' = H(s_K (.) q) * scale * log2(e) / sqrt(d), per (KV head, query head), into the workspace
//                 (only for the key-bias term with 1 or 2 padded query heads: otherwise the scores kernels
//                 compute it themselves)
//   attn_scores   one thread per token: scores in log2 units into LDS, chunk max m_c, p = 2^(s - m_c), l_c
//   attn_values   16 lanes per token: a_c = sum_t p_t n_t t[c_t] in the rotated domain
//   attn_combine  merges the chunks, divides by the softmax sum, inverse rotation, output and log-sum-exp
// With equal key and value bit widths attn_chunk runs the scores and values phases in one kernel and keeps the
// weights p in LDS (attn_scores and attn_values remain for unequal widths and for per-channel keys).
// Query heads of one KV head (grouped-query attention) share every table read; their count is padded to
// 1, 2, 4 or 8 (padded queries are zero and never written out). With 4 or 8 the scores' and the values' products
// run on the matrix cores (v_mfma_f32_4x4x1f32, below).
#include "pitch_device.h"

#ifndef PITCH_DIM
#error "compile with -DPITCH_DIM=<dim>"
#endif

namespace pitch {
namespace {

constexpr int kMaxChunk = 1024;          // tokens per workgroup; a chunk's scores stay in LDS
#ifndef PITCH_ATTN_FUSED
#define PITCH_ATTN_FUSED 1  // keys and values of equal bit width: scores and values in one kernel (attn_chunk)
#endif
#ifndef PITCH_ATTN_MFMA
#define PITCH_ATTN_MFMA 1  // four or eight query heads: their products on the matrix cores (below)
#endif
constexpr float kLn2 = 0x1.62e430p-1f;   // ln(2)

// Matrix-core products for four or eight query heads per KV head. v_mfma_f32_4x4x1f32 computes 16 independent
// 4 x 4 outer products per wave: D[v] of lane l += A(lane 4 (l / 4) + v) * B(lane l), in float32 (lane layout
// checked on gfx950 with lane-numbered operands). Scores: A = the token's table value (one token per lane), B = the
// rotated query of head l % 4 at the same coordinate, so D[v] of lane l accumulates the score of token
// 4 (l / 4) + v for head l % 4. Values: A = the token's weight for head l % 4, B = the table value of coordinate
// pair l of the token (d = 128: 64 pairs, one per lane; d = 64: lanes 32-63 take pair l - 32 of the next token),
// so D[v] of lane l accumulates head v's weighted sum of that coordinate. One instruction replaces four per-lane
// fmas at half their issue cycles, on a unit of its own.
typedef float v4f __attribute__((ext_vector_type(4)));
template <int NQ>
constexpr bool attn_mfma() { return PITCH_ATTN_MFMA && (NQ == 4 || NQ == 8); }
#ifndef PITCH_ATTN_QLDS
#define PITCH_ATTN_QLDS 1  // one or two query heads: rotated queries in LDS, read as broadcasts (no prep launch)
#endif
// Whether the scores kernels (without the key-bias term) rotate the queries themselves.
template <int NQ>
constexpr bool attn_rotates() { return attn_mfma<NQ>() || PITCH_ATTN_QLDS; }
__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}
// x of lane 4 (lane / 4) + V (a DPP quad broadcast)
template <int V>
__device__ __forceinline__ float quad_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), V * 0x55, 0xF, 0xF, true));
}
#ifndef PITCH_ATTN_VTOK
#define PITCH_ATTN_VTOK 8  // matrix-core values phase: tokens per step (4, 8 or 16)
#endif
constexpr int kQStride = 4;  // padding of an LDS query row (floats): rows stay 16-byte aligned

// Workspace regions (floats): rotated queries [kv][D/2][nqp][2], weights p [kv][T][nqp],
// chunk (max, sum) [kv][nqp][chunks][2], chunk accumulators [kv][nqp][chunks][D], and for key-bias removal the
// query products (q (.) b, q (.) rotate_half(b)) * scale * log2(e) as [kv][D][nqp][2].
struct WsLayout {
  uint64_t p, ml, acc, kbq;
  __host__ __device__ explicit WsLayout(const AttnArgs& a) {
    p = (uint64_t)a.kv_heads * a.dim * a.nqp;
    ml = p + (uint64_t)a.kv_heads * a.tokens * a.nqp;
    acc = ml + (uint64_t)a.kv_heads * a.nqp * a.chunks * 2;
    kbq = acc + (uint64_t)a.kv_heads * a.nqp * a.chunks * a.dim;
  }
};

// Value table of a code pair: codes c0 (bits [0, B)) and c1 (bits [B, 2B)) -> the two rotated-domain values
// their decode gives before the scale. B <= 5: one table of 2^(2B) float2. B >= 6: U[c0] * W[c1] element-wise
// from two 2^B-entry float2 tables (TurboQuant: U = (cb, 1), W = (1, cb); PolarQuant: U = (r, r),
// W = (cos, sin)). Built from the same constant tables as the decoders (gen_tables.py).
template <int D, int B>
struct PairLut {
  static constexpr int L = 1 << B;
  static constexpr bool kPair = B <= 5;
  static constexpr int N = kPair ? (1 << (2 * B)) : 2 * L;  // float2 entries

  __device__ static void build(float2* s, bool polar) {
    if (polar) {
      constexpr int off = pitch_polar_offset(B);
      const float* rad = pitch_polar_radius_tab + off;
      const float* cs = pitch_polar_cos_tab + off;
      const float* sn = pitch_polar_sin_tab + off;
      if constexpr (kPair) {
        for (int i = threadIdx.x; i < N; i += blockDim.x) {
          const float r = rad[i & (L - 1)];
          s[i] = make_float2(r * cs[i >> B], r * sn[i >> B]);
        }
      } else {
        for (int i = threadIdx.x; i < L; i += blockDim.x) {
          s[i] = make_float2(rad[i], rad[i]);
          s[L + i] = make_float2(cs[i], sn[i]);
        }
      }
    } else {
      const float* cb = pitch_codebook_tab + pitch_codebook_offset(ilog2(D), B);
      if constexpr (kPair) {
        for (int i = threadIdx.x; i < N; i += blockDim.x) s[i] = make_float2(cb[i & (L - 1)], cb[i >> B]);
      } else {
        for (int i = threadIdx.x; i < L; i += blockDim.x) {
          s[i] = make_float2(cb[i], 1.f);
          s[L + i] = make_float2(1.f, cb[i]);
        }
      }
    }
  }

  __device__ static float2 get(const float2* s, uint32_t bits) {
    if constexpr (kPair) {
      return s[bits & (uint32_t)(N - 1)];
    } else {
      const float2 u = s[bits & (uint32_t)(L - 1)], w = s[L + ((bits >> B) & (uint32_t)(L - 1))];
      return make_float2(u.x * w.x, u.y * w.y);
    }
  }
};

// One packed code row of NW words.
template <int NW>
__device__ __forceinline__ void load_row(const uint32_t* row, uint32_t (&w)[NW]) {
  int i = 0;
#pragma unroll
  for (; i + 4 <= NW; i += 4) {
    const u32x4 v = *(const u32x4*)(row + i);
    w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
  }
#pragma unroll
  for (; i + 2 <= NW; i += 2) {
    const u32x2 v = *(const u32x2*)(row + i);
    w[i] = v.x; w[i + 1] = v.y;
  }
}

// Sum or max over the 256 threads of a workgroup, per element; every thread gets the results.
template <int NQ, bool MAX>
__device__ __forceinline__ void block_reduce(float (&v)[NQ], float* s_red) {
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_xor(v[h], off);
      v[h] = MAX ? fmaxf(v[h], o) : v[h] + o;
    }
  }
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int h = 0; h < NQ; ++h) s_red[wid * NQ + h] = v[h];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const float a = s_red[h], b = s_red[NQ + h], c = s_red[2 * NQ + h], d = s_red[3 * NQ + h];
    v[h] = MAX ? fmaxf(fmaxf(a, b), fmaxf(c, d)) : (a + b) + (c + d);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------- prep
// One wave per (KV head, padded query head): q'' = H(s_K (.) q) * qscale, stored as [pair][query][2].
template <int D>
__global__ __launch_bounds__(64) void attn_prep(AttnArgs a) {
  constexpr int E = D / 64;
  const uint32_t kv = blockIdx.x / a.nqp, h = blockIdx.x % a.nqp;
  const int lane = threadIdx.x;
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane * E + e;
    const float x = h < a.nq ? a.q[((uint64_t)kv * a.nq + h) * D + j] : 0.f;
    v[e] = sign_is_negative(a.kseed, (uint32_t)j) ? -x : x;
  }
  fwht_contig<E, 64, float>(v, lane);
  float* qp = a.ws + (uint64_t)kv * D * a.nqp;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane * E + e;
    qp[((uint64_t)(j >> 1) * a.nqp + h) * 2 + (j & 1)] = v[e] * a.qscale;
  }
  if (a.kb_cos) {
    // q . o_t = sum_j (q_j b_j) cos_tj + (q_j rotate_half(b)_j) sin_tj, rotate_half(b)_j = -b_(j+D/2) for j < D/2
    // and b_(j-D/2) above; the products carry the scores' scale and log2(e)
    const float* bb = a.kb_bias + (uint64_t)kv * D;
    float* kq = a.ws + WsLayout(a).kbq + (uint64_t)kv * D * a.nqp * 2;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int j = lane * E + e;
      const float x = h < a.nq ? a.q[((uint64_t)kv * a.nq + h) * D + j] : 0.f;
      const float rh = j < D / 2 ? -bb[j + D / 2] : bb[j - D / 2];
      kq[((uint64_t)j * a.nqp + h) * 2] = x * bb[j] * a.kscale;
      kq[((uint64_t)j * a.nqp + h) * 2 + 1] = x * rh * a.kscale;
    }
  }
}

// Key-bias term of token t's scores for NQ queries, in log2 units: sum_j U_hj cos_tj + W_hj sin_tj over the row
// of position kb_first + t (U, W from attn_prep; their reads are wave-uniform), with two partial sums per query.
template <int D, int NQ>
__device__ __forceinline__ void key_bias_scores(const AttnArgs& a, const float* __restrict__ kq, uint64_t t,
                                                float (&bias)[NQ]) {
  const f32x4* cr = (const f32x4*)(a.kb_cos + (a.kb_first + t) * D);
  const f32x4* sr = (const f32x4*)(a.kb_sin + (a.kb_first + t) * D);
  float s0[NQ], s1[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) s0[h] = s1[h] = 0.f;
  for (int j4 = 0; j4 < D / 4; ++j4) {
    const f32x4 c4 = cr[j4], n4 = sr[j4];
    const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {n4.x, n4.y, n4.z, n4.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float* u = kq + (uint64_t)(4 * j4 + r) * NQ * 2;
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        float& acc = (r & 1) ? s1[h] : s0[h];
        acc = __builtin_fmaf(u[2 * h], cs[r], acc);
        acc = __builtin_fmaf(u[2 * h + 1], sn[r], acc);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < NQ; ++h) bias[h] = s0[h] + s1[h];
}

// ---------------------------------------------------------------------------------------------- scores
// Scores of chunk c of KV head kv, one thread per token, into s_s in log2 units; then the chunk maximum m, the
// weights p = 2^(s - m) and their sum l. (m, l) go to the workspace; the weights overwrite s_s, or with
// WRITE_P go to the workspace for a separate values kernel. The phase builds the key codes' pair table in s_tab.
// Without the key-bias term (attn_rotates) the phase computes the rotated queries itself into s_q (NQ rows of
// D + kQStride floats, 16-byte aligned, which nothing else uses until the phase ends) as [head][coordinate]:
// with four or eight query heads (attn_mfma) the products run on the matrix cores, with one or two each lane
// reads the query pairs from s_q (the same address in every lane: broadcast reads). With the key-bias term the
// rotated queries come from attn_prep through qp_all, whose wave-uniform reads can be scalar loads.
template <int D, int B, int NQ, bool WRITE_P, bool KB = false>
__device__ __forceinline__ void scores_phase(const AttnArgs& a, const float* __restrict__ qp_all, float2* s_tab,
                                             float* s_s, float* s_red, float* s_q, uint32_t kv, uint32_t c) {
  using P = PairLut<D, B>;
  constexpr int NW = D * B / 32;
  constexpr bool kMfma = attn_mfma<NQ>();
  // the phase rotates the queries into s_q (with the key-bias term only in the matrix-core form, which also
  // puts the bias products U = q (.) b and W = q (.) rotate_half(b), times kscale, in rows NQ .. 3 NQ - 1)
  constexpr bool kRot = attn_rotates<NQ>() && (!KB || kMfma);
  constexpr int QS = D + kQStride;
  const int tid = threadIdx.x;
  const uint64_t t0 = (uint64_t)c * a.chunk;
  const uint32_t n = (uint32_t)min((uint64_t)a.chunk, a.tokens - t0);
  const float* __restrict__ qp = qp_all + (uint64_t)kv * D * NQ;

  // software pipeline: the next token's code row and scale are loaded before this token's scores are computed
  auto fetch = [&](uint32_t i, uint32_t (&w)[NW], float& nk) {
    const uint64_t vi = (t0 + (i < n ? i : 0u)) * a.token_stride + (uint64_t)kv * a.head_stride;
    load_row<NW>(a.k_codes + vi * NW, w);
    nk = a.k_scales[vi];
  };
  uint32_t wn[NW];
  float nkn;
  fetch(tid, wn, nkn);
  // the pair table, its loads issued after the first code rows' (one barrier below covers table and queries)
  P::build(s_tab, a.kpolar != 0);
  if constexpr (kRot) {
    // the rotated queries, computed here as attn_prep computes them (no prep launch for these calls): wave w
    // rotates heads w and w + 4
    constexpr int E = D / 64;
    const int lane = tid & 63;
    for (int h = tid >> 6; h < NQ; h += kBlock / 64) {
      float v[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int j = lane * E + e;
        const float x = h < (int)a.nq ? a.q[((uint64_t)kv * a.nq + h) * D + j] : 0.f;
        v[e] = sign_is_negative(a.kseed, (uint32_t)j) ? -x : x;
        if constexpr (KB) {  // as attn_prep: rotate_half(b)_j = -b_(j+D/2) for j < D/2 and b_(j-D/2) above
          const float* bb = a.kb_bias + (uint64_t)kv * D;
          const float rh = j < D / 2 ? -bb[j + D / 2] : bb[j - D / 2];
          s_q[(NQ + h) * QS + j] = x * bb[j] * a.kscale;
          s_q[(2 * NQ + h) * QS + j] = x * rh * a.kscale;
        }
      }
      fwht_contig<E, 64, float>(v, lane);
#pragma unroll
      for (int e = 0; e < E; ++e) s_q[h * QS + lane * E + e] = v[e] * a.qscale;
    }
  }
  __syncthreads();
  for (uint32_t i0 = 0; i0 < n; i0 += kBlock) {
    const uint32_t i = i0 + tid;
    const bool valid = i < n;
    uint32_t w[NW];
#pragma unroll
    for (int k = 0; k < NW; ++k) w[k] = wn[k];
    const float nk = nkn;
    if (i0 + kBlock < n) fetch(i + kBlock, wn, nkn);
    if constexpr (kMfma) {
      const int lane = tid & 63;
      // key-bias term q . o_t = sum_j U_hj cos_tj + W_hj sin_tj on the matrix cores too: A = the cos or sin row
      // of the lane's token's position (a token past the chunk's end: its first), B = U or W of head l % 4
      v4f bc0 = {0.f, 0.f, 0.f, 0.f}, bs0 = bc0, bc1 = bc0, bs1 = bc0;
      if constexpr (KB) {
        const uint64_t pos = a.kb_first + t0 + (valid ? i : 0u);
        const f32x4* cr = (const f32x4*)(a.kb_cos + pos * D);
        const f32x4* sr = (const f32x4*)(a.kb_sin + pos * D);
        const float* u0 = s_q + (NQ + (lane & 3)) * QS;
        const float* w0 = s_q + (2 * NQ + (lane & 3)) * QS;
#pragma unroll 4
        for (int j4 = 0; j4 < D / 4; ++j4) {
          const f32x4 c4 = cr[j4], n4 = sr[j4];
          const v4f ua = *(const v4f*)(u0 + 4 * j4), wa = *(const v4f*)(w0 + 4 * j4);
          v4f ub = ua, wb = wa;
          if constexpr (NQ == 8) {
            ub = *(const v4f*)(u0 + 4 * QS + 4 * j4);
            wb = *(const v4f*)(w0 + 4 * QS + 4 * j4);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bc0 = mfma4(c4[r], ua[r], bc0);
            bs0 = mfma4(n4[r], wa[r], bs0);
            if constexpr (NQ == 8) {
              bc1 = mfma4(c4[r], ub[r], bc1);
              bs1 = mfma4(n4[r], wb[r], bs1);
            }
          }
        }
        // keeps the scores' LDS reads below: the scheduler otherwise issues all of them before these loads
        __builtin_amdgcn_sched_barrier(0);
      }
      // c (even coordinates) and e (odd ones): two independent chains per group of four heads
      const float* q0 = s_q + (lane & 3) * QS;
      v4f c0 = {0.f, 0.f, 0.f, 0.f}, e0 = c0, c1 = c0, e1 = c0;
#pragma unroll
      for (int p = 0; p < D / 2; p += 2) {
        const v4f qa = *(const v4f*)(q0 + 2 * p);  // coordinates 2p .. 2p + 3 of head lane % 4
        v4f qb = qa;
        if constexpr (NQ == 8) qb = *(const v4f*)(q0 + 4 * QS + 2 * p);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int pos = 2 * B * (p + u), wi = pos >> 5, sh = pos & 31;
          const uint32_t bits = (sh + 2 * B <= 32) ? (w[wi] >> sh) : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
          const float2 t = P::get(s_tab, bits);
          c0 = mfma4(t.x, qa[2 * u], c0);
          e0 = mfma4(t.y, qa[2 * u + 1], e0);
          if constexpr (NQ == 8) {
            c1 = mfma4(t.x, qb[2 * u], c1);
            e1 = mfma4(t.y, qb[2 * u + 1], e1);
          }
        }
      }
      // lane l holds the scores of tokens 4 (l / 4) + v for head l % 4 (and l % 4 + 4); each takes its token's scale
      const float nv[4] = {quad_bcast<0>(nk), quad_bcast<1>(nk), quad_bcast<2>(nk), quad_bcast<3>(nk)};
      const uint32_t ib = i0 + (uint32_t)(tid & ~3);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (ib + v < n) {
          s_s[(ib + v) * NQ + (lane & 3)] = __builtin_fmaf(c0[v] + e0[v], nv[v], bc0[v] + bs0[v]);
          if constexpr (NQ == 8)
            s_s[(ib + v) * NQ + 4 + (lane & 3)] = __builtin_fmaf(c1[v] + e1[v], nv[v], bc1[v] + bs1[v]);
        }
      }
      continue;
    }
    float acc[NQ];
#pragma unroll
    for (int h = 0; h < NQ; ++h) acc[h] = 0.f;
#pragma unroll
    for (int p = 0; p < D / 2; ++p) {
      const int pos = 2 * B * p, wi = pos >> 5, sh = pos & 31;
      const uint32_t bits = (sh + 2 * B <= 32) ? (w[wi] >> sh) : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
      const float2 t = P::get(s_tab, bits);
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        float2 q2;
        if constexpr (kRot) q2 = *(const float2*)(s_q + h * QS + 2 * p);  // the same address in every lane
        else q2 = make_float2(qp[(p * NQ + h) * 2], qp[(p * NQ + h) * 2 + 1]);
        acc[h] = __builtin_fmaf(q2.x, t.x, acc[h]);
        acc[h] = __builtin_fmaf(q2.y, t.y, acc[h]);
      }
    }
    if constexpr (KB) {  // key-bias removal: + q . o_t (position of a token past the chunk's end: its first)
      float kb[NQ];
      key_bias_scores<D, NQ>(a, a.ws + WsLayout(a).kbq + (uint64_t)kv * D * NQ * 2, t0 + (valid ? i : 0u), kb);
      if (valid) {
#pragma unroll
        for (int h = 0; h < NQ; ++h) s_s[i * NQ + h] = __builtin_fmaf(acc[h], nk, kb[h]);
      }
    } else if (valid) {
#pragma unroll
      for (int h = 0; h < NQ; ++h) s_s[i * NQ + h] = acc[h] * nk;
    }
  }
  __syncthreads();

  // chunk maximum, weights p = 2^(s - m) and their sum
  float m[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) m[h] = -__builtin_inff();
  for (uint32_t i = tid; i < n; i += kBlock) {
#pragma unroll
    for (int h = 0; h < NQ; ++h) m[h] = fmaxf(m[h], s_s[i * NQ + h]);
  }
  block_reduce<NQ, true>(m, s_red);
  const WsLayout L(a);
  float* pw = a.ws + L.p + ((uint64_t)kv * a.tokens + t0) * NQ;
  float l[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) l[h] = 0.f;
  for (uint32_t i = tid; i < n; i += kBlock) {
    float e[NQ];
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      e[h] = exp2f(s_s[i * NQ + h] - m[h]);
      l[h] += e[h];
    }
    float* dst = WRITE_P ? pw : s_s;  // each thread rewrites only the scores it read
    if constexpr (NQ % 4 == 0) {
#pragma unroll
      for (int h = 0; h < NQ; h += 4) *(f32x4*)(dst + (uint64_t)i * NQ + h) = f32x4{e[h], e[h + 1], e[h + 2], e[h + 3]};
    } else {
#pragma unroll
      for (int h = 0; h < NQ; ++h) dst[(uint64_t)i * NQ + h] = e[h];
    }
  }
  block_reduce<NQ, false>(l, s_red);  // its barriers also publish the weights in s_s
  if (tid == 0) {
    float* ml = a.ws + L.ml;
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const uint64_t k = (((uint64_t)kv * NQ + h) * a.chunks + c) * 2;
      ml[k] = m[h];
      ml[k + 1] = l[h];
    }
  }
}

// Workgroup (chunk, KV head); thread = token. KB: with the key-bias term (such calls always take these kernels).
template <int D, int B, int NQ, bool KB>
__global__ __launch_bounds__(kBlock) void attn_scores(AttnArgs a, const float* __restrict__ qp_all) {
  using P = PairLut<D, B>;
  __shared__ float2 s_tab[P::N];
  // the scores and, behind them, the query rows of the matrix-core form: one array, so that the compiler keeps the
  // query reads inside the token loop (from a separate array it hoists all D * NQ of them into registers)
  constexpr bool kRot = attn_rotates<NQ>() && (!KB || attn_mfma<NQ>());  // as in scores_phase
  __shared__ __attribute__((aligned(16))) float s_s[kMaxChunk * NQ + (kRot ? (KB ? 3 : 1) * NQ * (D + kQStride) : 0)];
  __shared__ float s_red[4 * NQ];
  scores_phase<D, B, NQ, true, KB>(a, qp_all, s_tab, s_s, s_red, s_s + kMaxChunk * NQ, blockIdx.y, blockIdx.x);
}

// ---------------------------------------------------------------------------------------------- scores, KIVI keys
// Per-channel keys decode as k_j = f32(c_j) * step_j + lo_j per group (reference/pitch_reference.py:165-174), so
// q . k_t = sum_j (q_j step_j) c_tj + sum_j q_j lo_j. Workgroup (chunk, KV head); thread = token; a wave's 64
// tokens lie in one group (the group size is a multiple of 64), so the wave builds that group's query products
// qs_j = q_j * step_j (times scale * log2 e) in its LDS slice and the per-query constant q . lo, then each lane
// reads its token's codes and sums qs_j * c_j with broadcast LDS reads. Chunk max, weights and sums as attn_scores.
template <int D, int B, int NQ>
__global__ __launch_bounds__(kBlock) void attn_scores_chan(AttnArgs a) {
  constexpr int NW = D * B / 32;
  constexpr int E = D / 64;                 // coordinates per lane when the wave builds the query products
  constexpr uint32_t kMask = (1u << B) - 1u;
  const float levels = (float)((1 << B) - 1);
  __shared__ float s_s[kMaxChunk * NQ];
  __shared__ float s_red[4 * NQ];
  // four or eight query heads: the products on the matrix cores (as in scores_phase), the query products per wave
  // as [query][coordinate] rows of D + kQStride; otherwise per-lane fmas over [coordinate][query]
  constexpr bool kM = attn_mfma<NQ>();
  constexpr int QS = D + kQStride;
  __shared__ __attribute__((aligned(16))) float s_qs[4][kM ? NQ * QS : D * NQ];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const uint32_t kv = blockIdx.y, c = blockIdx.x;
  const uint64_t t0 = (uint64_t)c * a.chunk;
  const uint32_t n = (uint32_t)min((uint64_t)a.chunk, a.tokens - t0);
  const uint64_t groups_per_head = a.head_stride / a.k_group;
  // this lane's query coordinates j = E * lane + e, scaled by scale * log2(e)
  float qv[NQ][E];
#pragma unroll
  for (int h = 0; h < NQ; ++h)
#pragma unroll
    for (int e = 0; e < E; ++e)
      qv[h][e] = h < (int)a.nq ? a.q[((uint64_t)kv * a.nq + h) * D + E * lane + e] * a.kscale : 0.f;
  float* qs = s_qs[wid];
  uint64_t cur_group = ~0ull;
  float beta[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) beta[h] = 0.f;

  for (uint32_t i0 = 0; i0 < n; i0 += kBlock) {
    const uint32_t wfirst = i0 + 64u * wid;   // this wave's first token in the chunk
    if (wfirst < n) {                          // uniform per wave
      const uint64_t g = (t0 + wfirst) / a.k_group;
      if (g != cur_group) {
        cur_group = g;
        const uint16_t* rg = a.k_ranges + ((uint64_t)kv * groups_per_head + g) * 2u * D;
#pragma unroll
        for (int h = 0; h < NQ; ++h) beta[h] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int j = E * lane + e;
          const float lo = widen1<1>(rg[j]), hi = widen1<1>(rg[D + j]);
          float step = (hi - lo) / levels;
          step = step == 0.f ? 1.f : step;
#pragma unroll
          for (int h = 0; h < NQ; ++h) {
            qs[kM ? h * QS + j : j * NQ + h] = qv[h][e] * step;
            beta[h] = __builtin_fmaf(qv[h][e], lo, beta[h]);
          }
        }
#pragma unroll
        for (int h = 0; h < NQ; ++h)
#pragma unroll
          for (int off = 1; off < 64; off <<= 1) beta[h] += __shfl_xor(beta[h], off);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      const uint32_t i = wfirst + lane;
      const bool valid = i < n;
      const uint64_t row = (uint64_t)kv * a.head_stride + t0 + (valid ? i : wfirst);
      uint32_t w[NW];
      load_row<NW>(a.k_codes + row * NW, w);
      if constexpr (kM) {
        // D[v] of lane l: token wfirst + 4 (l / 4) + v, head l % 4 (c: even coordinates, e: odd ones)
        const float* q0 = qs + (lane & 3) * QS;
        v4f c0 = {0.f, 0.f, 0.f, 0.f}, e0 = c0, c1 = c0, e1 = c0;
#pragma unroll
        for (int j = 0; j < D; j += 4) {
          const v4f qa = *(const v4f*)(q0 + j);
          v4f qb = qa;
          if constexpr (NQ == 8) qb = *(const v4f*)(q0 + 4 * QS + j);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int pos = B * (j + r), wi = pos >> 5, sh = pos & 31;
            const uint32_t bits = (sh + B <= 32) ? (w[wi] >> sh) : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
            const float cf = (float)(bits & kMask);
            if (r & 1) {
              e0 = mfma4(cf, qa[r], e0);
              if constexpr (NQ == 8) e1 = mfma4(cf, qb[r], e1);
            } else {
              c0 = mfma4(cf, qa[r], c0);
              if constexpr (NQ == 8) c1 = mfma4(cf, qb[r], c1);
            }
          }
        }
        const int hl = lane & 3;
        float b0 = beta[0], b1 = beta[NQ == 8 ? 4 : 0];
#pragma unroll
        for (int k = 1; k < 4; ++k) {
          b0 = hl == k ? beta[k] : b0;
          if constexpr (NQ == 8) b1 = hl == k ? beta[4 + k] : b1;
        }
        const uint32_t ib = wfirst + (uint32_t)(lane & ~3);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          if (ib + v < n) {
            s_s[(ib + v) * NQ + hl] = (c0[v] + e0[v]) + b0;
            if constexpr (NQ == 8) s_s[(ib + v) * NQ + 4 + hl] = (c1[v] + e1[v]) + b1;
          }
        }
        continue;
      }
      float acc[NQ];
#pragma unroll
      for (int h = 0; h < NQ; ++h) acc[h] = beta[h];
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const int pos = B * j, wi = pos >> 5, sh = pos & 31;
        const uint32_t bits = (sh + B <= 32) ? (w[wi] >> sh) : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
        const float cf = (float)(bits & kMask);
        float qj[NQ];
        if constexpr (NQ % 4 == 0) {
#pragma unroll
          for (int h = 0; h < NQ; h += 4) {
            const float4 v4 = *(const float4*)(qs + j * NQ + h);
            qj[h] = v4.x; qj[h + 1] = v4.y; qj[h + 2] = v4.z; qj[h + 3] = v4.w;
          }
        } else {
#pragma unroll
          for (int h = 0; h < NQ; ++h) qj[h] = qs[j * NQ + h];
        }
#pragma unroll
        for (int h = 0; h < NQ; ++h) acc[h] = __builtin_fmaf(qj[h], cf, acc[h]);
      }
      if (valid) {
#pragma unroll
        for (int h = 0; h < NQ; ++h) s_s[i * NQ + h] = acc[h];
      }
    }
  }
  __syncthreads();

  float m[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) m[h] = -__builtin_inff();
  for (uint32_t i = tid; i < n; i += kBlock) {
#pragma unroll
    for (int h = 0; h < NQ; ++h) m[h] = fmaxf(m[h], s_s[i * NQ + h]);
  }
  block_reduce<NQ, true>(m, s_red);
  const WsLayout L(a);
  float* pw = a.ws + L.p + ((uint64_t)kv * a.tokens + t0) * NQ;
  float l[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) l[h] = 0.f;
  for (uint32_t i = tid; i < n; i += kBlock) {
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const float e = exp2f(s_s[i * NQ + h] - m[h]);
      l[h] += e;
      pw[(uint64_t)i * NQ + h] = e;
    }
  }
  block_reduce<NQ, false>(l, s_red);
  if (tid == 0) {
    float* ml = a.ws + L.ml;
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const uint64_t k = (((uint64_t)kv * NQ + h) * a.chunks + c) * 2;
      ml[k] = m[h];
      ml[k + 1] = l[h];
    }
  }
}

// ---------------------------------------------------------------------------------------------- values
// a_c = sum_t p_t n_t t[c_t] over chunk c of KV head kv into the workspace. Per block of 256 tokens, each thread
// stages one token's code row and weights p * n in LDS; then lane (r, g) of wave w takes token
// 16 * step + 4 * w + r and the g-th 16th of its code pairs, accumulating its 2 * PPL coordinates for every
// query head. The weights p come from s_p (P_LDS, the fused kernel) or from the workspace. s_acc may alias
// s_code: it is written only after a barrier that ends the staging.
template <int D, int B>
struct ValuesLayout {
  static constexpr int NW = D * B / 32;
  static constexpr int RS = NW + 1;  // staged row stride in words (odd: consecutive rows start on other banks)
  static constexpr int kCodeWords = kBlock * RS + 4;
  static constexpr int WS = kBlock + 4;  // row stride of the weights staged as [head][token] (matrix-core form)
  template <int NQ>
  static constexpr int weight_floats() { return NQ * WS; }
};
// With four or eight query heads (matrix-core form) the weights are staged as [head][token], wave w
// takes tokens 64 w .. 64 w + 63 of the block PITCH_ATTN_VTOK at a time, and lane l holds code pair l of each
// token (d = 64: pair l mod 32 of every second token, from token l / 32): its matrix-core accumulators hold
// coordinates 2 (l mod D/2) and 2 (l mod D/2) + 1 of every head.
template <int D, int B, int NQ, bool P_LDS>
__device__ __forceinline__ void values_phase(const AttnArgs& a, const float2* s_tab, const float* s_p,
                                             uint32_t* s_code, float* s_w, float* s_acc, uint32_t kv, uint32_t c) {
  using P = PairLut<D, B>;
  constexpr int NW = ValuesLayout<D, B>::NW;
  constexpr int RS = ValuesLayout<D, B>::RS;
  constexpr int WS = ValuesLayout<D, B>::WS;
  constexpr bool kMfma = attn_mfma<NQ>();
  constexpr int TPI = 128 / D;  // matrix-core form: tokens per instruction (d = 64: lanes 32-63 take the second)
  constexpr int PPL = D / 32;        // code pairs per lane
  constexpr int LB = PPL * 2 * B;    // code bits per lane
  static_assert(LB <= 64, "a lane's codes fit two words after alignment");
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, r = lane >> 4, g = lane & 15;
  const uint64_t t0 = (uint64_t)c * a.chunk;
  const uint32_t n = (uint32_t)min((uint64_t)a.chunk, a.tokens - t0);
  const WsLayout L(a);
  const float* pw = P_LDS ? s_p : a.ws + L.p + ((uint64_t)kv * a.tokens + t0) * NQ;
  const int bit0 = g * LB, wlo = bit0 >> 5;
  const uint32_t sh = (uint32_t)(bit0 & 31);

  float acc[NQ][2 * PPL];
#pragma unroll
  for (int h = 0; h < NQ; ++h)
#pragma unroll
    for (int e = 0; e < 2 * PPL; ++e) acc[h][e] = 0.f;
  v4f m0 = {0.f, 0.f, 0.f, 0.f}, m1 = m0, m2 = m0, m3 = m0;  // matrix-core form: heads 0-3 and 4-7, x and y
  const int pl = lane % (D / 2), hi = lane / (D / 2);  // matrix-core form: code pair and token of the lane
  const int mw = (2 * B * pl) >> 5;
  const uint32_t msh = (uint32_t)((2 * B * pl) & 31);

  // software pipeline: each thread loads the code row, scale and weights of its token of the next block while
  // the current block is accumulated
  auto fetch = [&](uint32_t i, uint32_t (&w)[NW], float (&wt)[NQ]) {
    const bool valid = i < n;
    const uint32_t iv = valid ? i : 0u;
    const uint64_t vi = (t0 + iv) * a.token_stride + (uint64_t)kv * a.head_stride;
    load_row<NW>(a.v_codes + vi * NW, w);
    const float nv = valid ? a.v_scales[vi] : 0.f;
#pragma unroll
    for (int h = 0; h < NQ; ++h) wt[h] = pw[(uint64_t)iv * NQ + h] * nv;
  };
  uint32_t rown[NW];
  float wtn[NQ];
  fetch(tid, rown, wtn);
  for (uint32_t i0 = 0; i0 < n; i0 += kBlock) {
    __syncthreads();  // the previous block's readers are done (and, the first time, the table is built)
#pragma unroll
    for (int k = 0; k < NW; ++k) s_code[tid * RS + k] = rown[k];
#pragma unroll
    for (int h = 0; h < NQ; ++h) s_w[kMfma ? h * WS + tid : tid * NQ + h] = wtn[h];
    __syncthreads();
    if (i0 + kBlock < n) fetch(i0 + kBlock + tid, rown, wtn);
    const uint32_t nt = min((uint32_t)kBlock, n - i0);
    if constexpr (kMfma) {
      // every one of the block's 256 slots was staged (tokens past the end with weight 0), so the last group of
      // four may run past nt; the loop bounds are wave-uniform
      constexpr int VT = PITCH_ATTN_VTOK;  // tokens per step: their LDS reads are issued together
      static_assert(VT % 4 == 0 && 64 % VT == 0, "steps of whole weight quads within a wave's 64 tokens");
      const uint32_t s1 = min(64u * (uint32_t)wid + 64u, nt);
      for (uint32_t s0 = 64u * (uint32_t)wid; s0 < s1; s0 += VT) {
        v4f wa[VT / 4], wb[VT / 4];
#pragma unroll
        for (int k = 0; k < VT / 4; ++k) {
          wa[k] = *(const v4f*)(s_w + (lane & 3) * WS + s0 + 4 * k);
          wb[k] = wa[k];
          if constexpr (NQ == 8) wb[k] = *(const v4f*)(s_w + (4 + (lane & 3)) * WS + s0 + 4 * k);
        }
        float2 t[VT / TPI];
#pragma unroll
        for (int u = 0; u < VT / TPI; ++u) {
          // token s0 + TPI u + hi; row[1] exists: rows have a padding word
          const uint32_t* row = s_code + (s0 + TPI * u + hi) * RS + mw;
          t[u] = P::get(s_tab, __builtin_amdgcn_alignbit(row[1], row[0], msh));
        }
#pragma unroll
        for (int u = 0; u < VT / TPI; ++u) {
          const int k = TPI * u;  // the lane's token is s0 + k + hi
          const float w0 = (TPI == 2 && hi) ? wa[(k + 1) / 4][(k + 1) % 4] : wa[k / 4][k % 4];
          m0 = mfma4(w0, t[u].x, m0);
          m1 = mfma4(w0, t[u].y, m1);
          if constexpr (NQ == 8) {
            const float w1 = (TPI == 2 && hi) ? wb[(k + 1) / 4][(k + 1) % 4] : wb[k / 4][k % 4];
            m2 = mfma4(w1, t[u].x, m2);
            m3 = mfma4(w1, t[u].y, m3);
          }
        }
      }
      continue;
    }
    for (uint32_t s0 = 0; s0 < nt; s0 += 16) {
      const uint32_t tok = s0 + wid * 4 + r;
      if (tok < nt) {
        const uint32_t* row = s_code + tok * RS + wlo;
        const uint32_t w0 = row[0], w1 = row[1];
        const uint32_t x0 = __builtin_amdgcn_alignbit(w1, w0, sh);
        uint32_t x1 = 0u;  // bits [sh + 32, sh + 64) of the lane's window, needed when it holds over 32 bits
        if constexpr (LB > 32) x1 = __builtin_amdgcn_alignbit(row[2], w1, sh);
        float wt[NQ];
        if constexpr (NQ % 4 == 0) {
#pragma unroll
          for (int h = 0; h < NQ; h += 4) {
            const float4 q4 = *(const float4*)(s_w + tok * NQ + h);
            wt[h] = q4.x; wt[h + 1] = q4.y; wt[h + 2] = q4.z; wt[h + 3] = q4.w;
          }
        } else {
#pragma unroll
          for (int h = 0; h < NQ; ++h) wt[h] = s_w[tok * NQ + h];
        }
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
          constexpr int W2 = 2 * B;
          const int o = W2 * j;
          const uint32_t bits = (o + W2 <= 32) ? (x0 >> o)
                                : (o >= 32 ? (x1 >> (o - 32)) : __builtin_amdgcn_alignbit(x1, x0, (uint32_t)o));
          const float2 t = P::get(s_tab, bits);
#pragma unroll
          for (int h = 0; h < NQ; ++h) {
            acc[h][2 * j] = __builtin_fmaf(wt[h], t.x, acc[h][2 * j]);
            acc[h][2 * j + 1] = __builtin_fmaf(wt[h], t.y, acc[h][2 * j + 1]);
          }
        }
      }
    }
  }
  if constexpr (kMfma) {
    if constexpr (TPI == 2) {  // lanes l and l + 32 summed different tokens of the same coordinates
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        m0[v] += __shfl_xor(m0[v], 32);
        m1[v] += __shfl_xor(m1[v], 32);
        if constexpr (NQ == 8) {
          m2[v] += __shfl_xor(m2[v], 32);
          m3[v] += __shfl_xor(m3[v], 32);
        }
      }
    }
    __syncthreads();  // staging reads are done (s_acc may alias s_code)
    if (hi == 0) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        *(float2*)(s_acc + (wid * NQ + v) * D + 2 * pl) = make_float2(m0[v], m1[v]);
        if constexpr (NQ == 8) *(float2*)(s_acc + (wid * NQ + 4 + v) * D + 2 * pl) = make_float2(m2[v], m3[v]);
      }
    }
  } else {
    // sum over the four token rows of the wave (lanes g, g + 16, g + 32, g + 48), then over the waves
#pragma unroll
    for (int h = 0; h < NQ; ++h)
#pragma unroll
      for (int e = 0; e < 2 * PPL; ++e) {
        acc[h][e] += __shfl_xor(acc[h][e], 16);
        acc[h][e] += __shfl_xor(acc[h][e], 32);
      }
    __syncthreads();  // staging reads are done (s_acc may alias s_code)
    if (r == 0) {
#pragma unroll
      for (int h = 0; h < NQ; ++h)
#pragma unroll
        for (int e = 0; e < 2 * PPL; ++e) s_acc[(wid * NQ + h) * D + 2 * PPL * g + e] = acc[h][e];
    }
  }
  __syncthreads();
  float* A = a.ws + L.acc;
  for (int x = tid; x < NQ * D; x += kBlock) {
    const int h = x / D, j = x % D;
    const float v = (s_acc[h * D + j] + s_acc[(NQ + h) * D + j]) + (s_acc[(2 * NQ + h) * D + j] + s_acc[(3 * NQ + h) * D + j]);
    A[(((uint64_t)kv * NQ + h) * a.chunks + c) * D + j] = v;
  }
}

// Workgroup (chunk, KV head), weights from the workspace.
template <int D, int B, int NQ>
__global__ __launch_bounds__(kBlock) void attn_values(AttnArgs a) {
  using P = PairLut<D, B>;
  __shared__ float2 s_tab[P::N];
  __shared__ uint32_t s_code[ValuesLayout<D, B>::kCodeWords];
  __shared__ __attribute__((aligned(16))) float s_w[ValuesLayout<D, B>::template weight_floats<NQ>()];
  __shared__ float s_acc[4 * NQ * D];
  P::build(s_tab, a.vpolar != 0);
  values_phase<D, B, NQ, false>(a, s_tab, nullptr, s_code, s_w, s_acc, blockIdx.y, blockIdx.x);
}

// ---------------------------------------------------------------------------------------------- scores + values
// One workgroup per (chunk, KV head) for keys and values of the same bit width: the scores phase leaves the
// chunk's weights p in LDS and the values phase reads them there, so p never goes through HBM and the call
// has one launch fewer. Dynamic LDS: [chunk * NQ] weights, then the values staging (codes and weights), whose
// space also holds the four waves' partial accumulators at the end.
template <int D, int B, int NQ>
struct FusedLds {
  static constexpr int kStageBytes =
      ValuesLayout<D, B>::kCodeWords * 4 + ValuesLayout<D, B>::template weight_floats<NQ>() * 4;
  static constexpr int kAccBytes = 4 * NQ * D * 4;
  static constexpr int kRegionBytes = kStageBytes > kAccBytes ? kStageBytes : kAccBytes;
  static constexpr int kStaticBytes = PairLut<D, B>::N * 8 + 4 * NQ * 4;
  static uint32_t dynamic_bytes(uint32_t chunk) { return chunk * NQ * 4u + (uint32_t)kRegionBytes; }
};
template <int D, int B, int NQ>
__global__ __launch_bounds__(kBlock) void attn_chunk(AttnArgs a, const float* __restrict__ qp_all) {
  using P = PairLut<D, B>;
  __shared__ float2 s_tab[P::N];
  __shared__ float s_red[4 * NQ];
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  float* s_s = s_dyn;                                       // a.chunk * NQ floats (a multiple of 16 bytes)
  uint32_t* s_code = (uint32_t*)(s_dyn + (size_t)a.chunk * NQ);
  float* s_w = (float*)(s_code + ValuesLayout<D, B>::kCodeWords);  // 16-byte aligned: kCodeWords % 4 == 0
  static_assert(ValuesLayout<D, B>::kCodeWords % 4 == 0, "weights staging stays 16-byte aligned");
  // the query rows of the scores phase use the values staging space, which is free until then
  static_assert(NQ * (D + kQStride) <= ValuesLayout<D, B>::kCodeWords, "query rows fit the staging space");
  scores_phase<D, B, NQ, false>(a, qp_all, s_tab, s_s, s_red, (float*)s_code, blockIdx.y, blockIdx.x);
  // the scores phase ended with a barrier after its last table read; the values phase begins with one
  if (a.vpolar != a.kpolar) P::build(s_tab, a.vpolar != 0);
  values_phase<D, B, NQ, true>(a, s_tab, s_s, s_code, s_w, (float*)s_code, blockIdx.y, blockIdx.x);
}

// ---------------------------------------------------------------------------------------------- combine
// Workgroup per (KV head, real query head): merges the chunks' (m, l, a), then o = s_V (.) H(a / l) / sqrt(d)
// and lse = (M + log2 l) * ln 2.
template <int D>
__global__ __launch_bounds__(kBlock) void attn_combine(AttnArgs a) {
  constexpr int E = D / 64;
  __shared__ float s_red[4];
  __shared__ float s_part[4 * (D + 1)];
  const uint32_t kv = blockIdx.x / a.nq, h = blockIdx.x % a.nq;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const WsLayout L(a);
  const float* ml = a.ws + L.ml + ((uint64_t)kv * a.nqp + h) * a.chunks * 2;
  const float* A = a.ws + L.acc + ((uint64_t)kv * a.nqp + h) * a.chunks * D;
  float M = -__builtin_inff();
  for (uint32_t c = tid; c < a.chunks; c += kBlock) M = fmaxf(M, ml[2 * c]);
  for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
  if (lane == 0) s_red[wid] = M;
  __syncthreads();
  M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  float ls = 0.f, acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  // chunks c = wid, wid + 4, ...; loads are issued kU chunks at a time so they overlap
  constexpr int kU = 16;
  for (uint32_t c0 = wid; c0 < a.chunks; c0 += 4 * kU) {
    float mv[kU], lv[kU], av[kU][E];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint32_t c = c0 + 4 * u;
      const bool in = c < a.chunks;
      const uint32_t cc = in ? c : c0;
      mv[u] = in ? ml[2 * cc] : -__builtin_inff();
      lv[u] = ml[2 * cc + 1];
#pragma unroll
      for (int e = 0; e < E; ++e) av[u][e] = A[(uint64_t)cc * D + lane * E + e];
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const float f = exp2f(mv[u] - M);  // 0 for chunks past the end
      ls = __builtin_fmaf(lv[u], f, ls);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = __builtin_fmaf(av[u][e], f, acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) s_part[wid * (D + 1) + lane * E + e] = acc[e];
  if (lane == 0) s_part[wid * (D + 1) + D] = ls;
  __syncthreads();
  if (wid != 0) return;  // no barrier follows
  float y[E];
  const float lsum = (s_part[D] + s_part[(D + 1) + D]) + (s_part[2 * (D + 1) + D] + s_part[3 * (D + 1) + D]);
  const float inv = 1.f / lsum;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane * E + e;
    y[e] = ((s_part[j] + s_part[(D + 1) + j]) + (s_part[2 * (D + 1) + j] + s_part[3 * (D + 1) + j])) * inv;
  }
  fwht_contig<E, 64, float>(y, lane);
  float* out = a.out + ((uint64_t)kv * a.nq + h) * D;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int j = lane * E + e;
    const float o = y[e] * a.oscale;
    out[j] = sign_is_negative(a.vseed, (uint32_t)j) ? -o : o;
  }
  if (lane == 0 && a.lse) a.lse[(uint64_t)kv * a.nq + h] = (M + log2f(lsum)) * kLn2;
}

template <int NQ, int B>
bool launch_fused(const AttnArgs& a, hipStream_t s) {
  using F = FusedLds<PITCH_DIM, B, NQ>;
  const uint32_t bytes = F::dynamic_bytes(a.chunk);
  if (bytes + (uint32_t)F::kStaticBytes > 65536u) return false;  // stay within 64 KB of LDS per workgroup
  hipLaunchKernelGGL((attn_chunk<PITCH_DIM, B, NQ>), dim3(a.chunks, a.kv_heads), dim3(kBlock), bytes, s, a,
                     (const float*)a.ws);
  return true;
}

template <int NQ>
hipError_t launch_nq(const AttnArgs& a, hipStream_t s) {
  constexpr int D = PITCH_DIM;
  const dim3 grid(a.chunks, a.kv_heads);
  const float* qp = a.ws;
  if (!a.k_ranges && !a.kb_cos && a.kbits == a.vbits && PITCH_ATTN_FUSED) {
    bool done = false;
    switch (a.kbits) {
#define PITCH_FUSED(B) \
  case B: done = launch_fused<NQ, B>(a, s); break;
      PITCH_FUSED(2) PITCH_FUSED(3) PITCH_FUSED(4) PITCH_FUSED(5) PITCH_FUSED(6) PITCH_FUSED(7) PITCH_FUSED(8)
#undef PITCH_FUSED
      default: return hipErrorInvalidValue;
    }
    if (done) return hipSuccess;
  }
  if (a.k_ranges) {
    switch (a.kbits) {
#define PITCH_SCORES_CHAN(B) \
  case B: hipLaunchKernelGGL((attn_scores_chan<D, B, NQ>), grid, dim3(kBlock), 0, s, a); break;
      PITCH_SCORES_CHAN(2) PITCH_SCORES_CHAN(3) PITCH_SCORES_CHAN(4) PITCH_SCORES_CHAN(5) PITCH_SCORES_CHAN(6)
      PITCH_SCORES_CHAN(7) PITCH_SCORES_CHAN(8)
#undef PITCH_SCORES_CHAN
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (a.kbits) {
#define PITCH_SCORES(B)                                                                          \
  case B:                                                                                        \
    if (a.kb_cos) hipLaunchKernelGGL((attn_scores<D, B, NQ, true>), grid, dim3(kBlock), 0, s, a, qp); \
    else hipLaunchKernelGGL((attn_scores<D, B, NQ, false>), grid, dim3(kBlock), 0, s, a, qp);        \
    break;
      PITCH_SCORES(2) PITCH_SCORES(3) PITCH_SCORES(4) PITCH_SCORES(5) PITCH_SCORES(6) PITCH_SCORES(7) PITCH_SCORES(8)
#undef PITCH_SCORES
      default: return hipErrorInvalidValue;
    }
  }
  switch (a.vbits) {
#define PITCH_VALUES(B) \
  case B: hipLaunchKernelGGL((attn_values<D, B, NQ>), grid, dim3(kBlock), 0, s, a); break;
    PITCH_VALUES(2) PITCH_VALUES(3) PITCH_VALUES(4) PITCH_VALUES(5) PITCH_VALUES(6) PITCH_VALUES(7) PITCH_VALUES(8)
#undef PITCH_VALUES
    default: return hipErrorInvalidValue;
  }
  return hipSuccess;
}

}  // namespace

#define PITCH_CAT2(a, b) a##b
#define PITCH_CAT(a, b) PITCH_CAT2(a, b)

hipError_t PITCH_CAT(launch_attention_d, PITCH_DIM)(const AttnArgs& a, hipStream_t s) {
  constexpr int D = PITCH_DIM;
  static_assert(D == 64 || D == 128, "attention dimensions");
  if (a.dim != (uint32_t)D || a.chunk < 64 || a.chunk > (uint32_t)kMaxChunk || a.chunks == 0) return hipErrorInvalidValue;
  if (a.k_ranges && (a.k_group == 0 || a.k_group % 64 != 0 || a.head_stride % a.k_group != 0 || a.token_stride != 1))
    return hipErrorInvalidValue;
  if (a.kb_cos && (a.k_ranges || !a.kb_bias || !a.kb_sin)) return hipErrorInvalidValue;
  // the scores kernels rotate the queries themselves (attn_rotates), with the key-bias term only in the
  // matrix-core form (attn_mfma)
  const bool rotate_inside = (a.nqp == 1 && attn_rotates<1>()) || (a.nqp == 2 && attn_rotates<2>()) ||
                             (a.nqp == 4 && attn_rotates<4>()) || (a.nqp == 8 && attn_rotates<8>());
  const bool mfma = (a.nqp == 4 && attn_mfma<4>()) || (a.nqp == 8 && attn_mfma<8>());
  if (!a.k_ranges && !(rotate_inside && (!a.kb_cos || mfma)))
    hipLaunchKernelGGL((attn_prep<D>), dim3(a.kv_heads * a.nqp), dim3(64), 0, s, a);
  hipError_t e;
  switch (a.nqp) {
    case 1: e = launch_nq<1>(a, s); break;
    case 2: e = launch_nq<2>(a, s); break;
    case 4: e = launch_nq<4>(a, s); break;
    case 8: e = launch_nq<8>(a, s); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_combine<D>), dim3(a.kv_heads * a.nq), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

}  // namespace pitch
