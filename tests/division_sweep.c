/* Randomised sweep of the per-channel encoder's division-free quotient against correctly rounded float32
 * division (reference/pitch_reference.py:155-158 computes step = (hi - lo) / (2^b - 1) and
 * floor((x - lo) / step + 0.5) in float32).
 *
 *   step:     s0 = RN(d * RN(1/L)),  step = RN(s0 + (d - s0*L) * RN(1/L))      (fmaf twice)
 *   quotient: q0 = RN(a * inv),      q = RN(q0 + (a - q0*min(step, FLT_MAX)) * inv), inv = RN(1/step)
 *
 * Operands come from the codec's domain: hi > lo are fp16 values, L = 2^b - 1 for b = 1..8, and x lies inside
 * [lo, hi] widened by the rounding of the true extremes to fp16, drawn uniformly, at the ends and next to
 * every rounding point of t = q + 0.5. Prints the counts and exits 1 if any code differs, or any quotient
 * differs other than a subnormal one (whose code is 0 either way) or a step that is a signed zero.
 * Usage: division_sweep <ranges>   (each range is checked with 8 values)
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t state = 88172645463325252ull;
static uint64_t next(void) {
  state ^= state << 13;
  state ^= state >> 7;
  state ^= state << 17;
  return state;
}
static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float half_to_float(uint16_t h) {  /* finite fp16 only */
  const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 0) { const float v = ldexpf((float)m, -24); return sign ? -v : v; }
  return from_bits(sign | ((e + 112u) << 23) | (m << 13));
}

int main(int argc, char** argv) {
  const long n = argc > 1 ? atol(argv[1]) : 1000000;
  long tested = 0, quotient_diff = 0, code_diff = 0, step_diff = 0;
  for (long i = 0; i < n; ++i) {
    const uint16_t h1 = (uint16_t)(next() & 0xffffu), h2 = (uint16_t)(next() & 0xffffu);
    if (((h1 >> 10) & 31u) == 31u || ((h2 >> 10) & 31u) == 31u) continue;
    float lo = half_to_float(h1), hi = half_to_float(h2);
    if (lo > hi) { const float t = lo; lo = hi; hi = t; }
    const float L = (float)((1 << (1 + (int)(next() % 8u))) - 1);
    const float il = 1.0f / L;
    const float d = hi - lo;
    const float s0 = d * il;
    const float sq = fmaf(fmaf(-s0, L, d), il, s0);
    if (to_bits(sq) != to_bits(d / L) && !(sq == 0.0f && d / L == 0.0f)) ++step_diff;
    const float step = sq == 0.0f ? 1.0f : sq;
    const float inv = 1.0f / step, stc = fminf(step, 0x1.fffffep127f);
    const float glo = nextafterf(lo, -INFINITY), ghi = nextafterf(hi, INFINITY);
    for (int j = 0; j < 8; ++j) {
      float x;
      const float k = (float)(next() % 512u) * 0.5f;
      switch (next() % 4u) {
        case 0: x = lo + (hi - lo) * (float)((next() >> 11) * 0x1.0p-53); break;
        case 1: x = lo + (k - 0.5f) * step; break;
        case 2: x = from_bits(to_bits(lo + k * step) + (uint32_t)(next() % 9u) - 4u); break;
        default: x = (next() & 1u) ? glo : ghi; break;
      }
      if (!isfinite(x) || x < glo || x > ghi) continue;
      const float a = x - lo;
      const float ref = a / step;
      const float q0 = a * inv;
      const float q = fmaf(fmaf(-q0, stc, a), inv, q0);
      ++tested;
      if (to_bits(q) != to_bits(ref) && !(fabsf(ref) < 0x1.0p-126f)) ++quotient_diff;
      const float c_ref = fminf(fmaxf(floorf(ref + 0.5f), 0.0f), L);
      const float c_q = fminf(fmaxf(floorf(q + 0.5f), 0.0f), L);
      if (c_ref != c_q) ++code_diff;
    }
  }
  printf("tested %ld quotient_diff %ld code_diff %ld step_diff %ld\n", tested, quotient_diff, code_diff, step_diff);
  return (quotient_diff || code_diff || step_diff) ? 1 : 0;
}
