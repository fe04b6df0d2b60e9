// frx_policy.hpp — host-side sizing rules of the context workspaces, kept
// free of HIP so that a CPU build can check them.
#pragma once
#include <stddef.h>

namespace frx {

// Size to allocate when a workspace of `have` bytes must hold `need`:
// at least 1.5x the old size (rounded to 256 bytes), so that a run of rising
// requests makes O(log(max / first)) allocations and the buffers it retires
// sum to less than twice the final size.
inline size_t grow_bytes(size_t have, size_t need) {
  const size_t a = (need + 255) & ~(size_t)255;
  if (need <= have) return have;
  const size_t g = have + have / 2;
  const size_t b = (g + 255) & ~(size_t)255;
  return b > a ? b : a;
}

}  // namespace frx
