/* Seeded synthetic inputs for bench.py and tests: the C twin of
 * quixicore_hip/synth.py (same splitmix64 counter stream, same Box-Muller
 * pairing), parallel over OpenMP threads.  Not part of the HIP library. */
#include <math.h>
#include <stdint.h>

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline double unit(uint64_t seed, uint64_t i) {
  return (double)(mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull) >> 40) * 0x1p-24;
}

void qcs_uniform(uint64_t seed, long long count, double* out) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < count; ++i) out[i] = unit(seed, (uint64_t)i);
}

void qcs_normal(uint64_t seed, long long count, double sigma, float* out) {
  const long long pairs = (count + 1) / 2;
#pragma omp parallel for schedule(static)
  for (long long p = 0; p < pairs; ++p) {
    const double u0 = unit(seed, (uint64_t)(2 * p));
    const double u1 = unit(seed, (uint64_t)(2 * p + 1));
    const double r = sqrt(-2.0 * log1p(-u0));
    const double t = 2.0 * 3.141592653589793 * u1;
    out[2 * p] = (float)(r * cos(t) * sigma);
    if (2 * p + 1 < count) out[2 * p + 1] = (float)(r * sin(t) * sigma);
  }
}
