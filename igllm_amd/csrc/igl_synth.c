/* igl_synth.c - the seeded synthetic inputs every measurement and parity test
 * uses, in portable C so the CPU and GPU hosts draw the same numbers.
 *
 * splitmix64 expands the seed into xoshiro256** state (Vigna's published
 * generators); normals are Box-Muller pairs in double precision from two
 * 53-bit uniforms, the first taken from (0, 1] so the logarithm is finite.
 */
#include <math.h>

#include "igl_backend.h"

static uint64_t splitmix64(uint64_t *x) {
  uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void igl_rng_seed(igl_rng *rng, uint64_t seed) {
  uint64_t x = seed;
  for (int i = 0; i < 4; ++i) rng->s[i] = splitmix64(&x);
}

uint64_t igl_rng_next(igl_rng *rng) {
  uint64_t *s = rng->s;
  const uint64_t result = rotl(s[1] * 5u, 7) * 9u;
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl(s[3], 45);
  return result;
}

void igl_rng_normal(igl_rng *rng, float *out, size_t count, float mean, float stddev) {
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < count) {
    double u1 = (double)((igl_rng_next(rng) >> 11) + 1u) * 0x1.0p-53;
    double u2 = (double)(igl_rng_next(rng) >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    out[i++] = (float)(mean + stddev * r * cos(two_pi * u2));
    if (i < count) out[i++] = (float)(mean + stddev * r * sin(two_pi * u2));
  }
}

void igl_rng_codes4(igl_rng *rng, uint8_t *codes, int N, int K, size_t row_stride) {
  for (int n = 0; n < N; ++n) {
    uint8_t *row = codes + (size_t)n * row_stride;
    for (int k = 0; k < K; k += 2) {
      uint8_t lo = (uint8_t)(igl_rng_next(rng) >> 60);
      uint8_t hi = k + 1 < K ? (uint8_t)(igl_rng_next(rng) >> 60) : 0u;
      row[k / 2] = (uint8_t)(lo | (hi << 4));
    }
    for (size_t b = (size_t)(K + 1) / 2; b < row_stride; ++b) row[b] = 0;
  }
}

void igl_rng_gains(igl_rng *rng, float *gains, size_t count, float stddev) {
  igl_rng_normal(rng, gains, count, 0.0f, stddev);
  for (size_t i = 0; i < count; ++i) gains[i] = fabsf(gains[i]);
}
