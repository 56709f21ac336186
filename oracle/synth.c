/* The reference's synthetic checkpoint values, restated from internal/llm/synth.go:17-35
 * (Synthetic.Get). Test infrastructure only (see oracle.h). */
#include "oracle.h"

/* or_fnv64a (qwen3.c) is Go's hash/fnv New64a, the seed of synth.go:23-25.
 * synth.go:27-33: seed = seed*6364136223846793005 + 1442695040888963407 before each element;
 * v = float32(int64(seed>>40) - (1<<23)) / (1<<23) * 0.2, each step a float32 operation */
void or_synth_reference(const char *name, size_t n, float *out) {
  uint64_t seed = or_fnv64a(name);
  for (size_t i = 0; i < n; i++) {
    seed = seed * 6364136223846793005ull + 1442695040888963407ull;
    float v = (float)((int64_t)(seed >> 40) - (1 << 23));
    v = v / 8388608.0f;
    out[i] = v * 0.2f;
  }
}
