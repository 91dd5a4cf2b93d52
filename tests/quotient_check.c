/*
 * The quantizer kernels (loractl_amd/csrc/lrq_quant.hip, k_quantize) form
 * RN(v / s) without a division per value: y = RN(1 / s), q0 = RN(v * y),
 * r = fma(-q0, s, v), RN(q0 + r * y) = fma(r, y, q0). This program checks
 * that sequence, written here with the C library's fmaf, against the
 * correctly rounded division on the kernels' domain (|v| <= 127.5 s, the
 * scales s = amax / 7 or amax / 127 for s >= 2^-80):
 *   - the quotient must equal RN(v / s) whenever |v / s| >= 2^-8;
 *   - round-half-away of it must equal round-half-away of RN(v / s) always.
 * Default: every f32 within 64 ulps of each rounding threshold (k + 1/2) s,
 * k = 0 .. 127, and 256 random v, for each of 4000 random scales. With
 * --exhaustive: every f32 v in the domain, for 24 scales (minutes, 8 cores).
 * Exit status 0 when nothing differs.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t ubits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static uint32_t next(void) {
  rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
  return (uint32_t)(rng >> 32);
}

static uint64_t bad_q, bad_r, total;

static void check(float v, float s, float y) {
  const float ref = v / s;
  const float q0 = v * y;
  const float r = fmaf(-q0, s, v);
  const float q = fmaf(r, y, q0);
  ++total;
  if (fabsf(ref) >= 0x1p-8f && q != ref) ++bad_q;
  if (roundf(q) != roundf(ref)) ++bad_r;
}

static float random_scale(void) {
  /* amax with an exponent from 2^-73 to 2^27, then / 7 or / 127 */
  const uint32_t e = 54 + next() % 101;
  const float amax = bits((next() & 0x007fffffu) | (e << 23));
  return (next() & 1) ? amax / 7.0f : amax / 127.0f;
}

int main(int argc, char** argv) {
  const int exhaustive = argc > 1 && strcmp(argv[1], "--exhaustive") == 0;
  const int scales = exhaustive ? 24 : 4000;
  for (int i = 0; i < scales; ++i) {
    const float s = random_scale();
    if (s < 0x1p-80f) continue;  /* the kernels divide there */
    const float y = 1.0f / s;
    if (exhaustive) {
      const uint32_t top = ubits(127.5f * s);
#pragma omp parallel for reduction(+ : bad_q, bad_r, total) schedule(static)
      for (int64_t u = 0; u <= (int64_t)top; ++u) {
        const float v = bits((uint32_t)u);
        const float ref = v / s, q0 = v * y, r = fmaf(-q0, s, v), q = fmaf(r, y, q0);
        ++total;
        if (fabsf(ref) >= 0x1p-8f && q != ref) ++bad_q;
        if (roundf(q) != roundf(ref)) ++bad_r;
      }
      continue;
    }
    for (int k = 0; k < 128; ++k) {
      const uint32_t c = ubits((k + 0.5f) * s);
      for (int d = -64; d <= 64; ++d) {
        check(bits(c + d), s, y);
        check(-bits(c + d), s, y);
      }
    }
    for (int j = 0; j < (1 << 8); ++j) {
      const float v = (float)((int)(next() % 255001u) - 127500) * 1e-3f * s;
      check(v, s, y);
    }
  }
  printf("checked %llu quotients: %llu differ (|v/s| >= 2^-8), %llu round differently\n",
         (unsigned long long)total, (unsigned long long)bad_q, (unsigned long long)bad_r);
  return (bad_q || bad_r) ? 1 : 0;
}
