/* C restatement of the seeded synthetic generator (test infrastructure only).
 * Same definition as oracle/synth.py; built by oracle/Makefile. */
#include <stdint.h>
#include <string.h>

static const uint64_t G = 0x9E3779B97F4A7C15ull;
static const uint32_t SCALE[3] = {0x350DE3BDu, 0x32E305FBu, 0x2DE878D0u};

static uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* kind: 0 param (bf16 bits in the low half), 1 main, 2 exp_avg, 3 exp_avg_sq. */
void oracle_synth(uint64_t seed, uint32_t param_id, uint32_t kind, const uint64_t *idx, uint64_t n,
                  uint32_t *out) {
  const uint32_t stream = kind <= 1 ? 0 : kind - 1;
  const uint64_t key = mix(mix(seed + G) + (4ull * param_id + stream + 1) * G);
  float scale;
  memcpy(&scale, &SCALE[stream], 4);
  /* Every element is independent: large requests are split over the host's threads. */
#pragma omp parallel for schedule(static) if (n > (1u << 16))
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t h = mix(key + (idx[i] + 1) * G);
    const int32_t s = (int32_t)((h & 0xffff) + ((h >> 16) & 0xffff) + ((h >> 32) & 0xffff) + (h >> 48)) - 131070;
    volatile float v = (float)s * scale;
    uint32_t b;
    memcpy(&b, (const void *)&v, 4);
    if (kind == 3) b &= 0x7fffffffu;
    if (kind <= 1) {
      const uint32_t bf = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
      b = kind == 0 ? bf : bf << 16;
    }
    out[i] = b;
  }
}
