// Host check of the workspace growth rule (frx::grow_bytes): rising
// requests make O(log) allocations and the retired buffers stay below twice
// the final size. Built with g++ by tests/test_c_abi.py; no GPU.
#include <stdio.h>

#include "frx_policy.hpp"

static int check(size_t first, size_t last, size_t step) {
  size_t have = 0, retired = 0;
  unsigned allocs = 0;
  for (size_t need = first; need <= last; need += step) {
    const size_t b = frx::grow_bytes(have, need);
    if (b < need || b % 256 != 0) {
      printf("grow_bytes(%zu, %zu) = %zu\n", have, need, b);
      return 1;
    }
    if (b != have) {
      retired += have;
      have = b;
      allocs++;
    }
  }
  // 1.5x growth: at most log_1.5(last / first) + 2 allocations
  unsigned bound = 2;
  for (double r = (double)last / (double)first; r > 1.0; r /= 1.5) bound++;
  if (allocs > bound || retired >= 2 * have) {
    printf("first %zu last %zu step %zu: %u allocations (bound %u), retired %zu of %zu\n", first, last, step, allocs,
           bound, retired, have);
    return 1;
  }
  return 0;
}

int main() {
  int bad = 0;
  // prefill M = 17..2048 at I = 11008 (fp32 h rows), and byte-sized steps
  bad |= check(17 * 11008 * 4, 2048 * 11008 * 4, 11008 * 4);
  bad |= check(1, 1 << 20, 1);
  bad |= check(256, 256 << 20, 4096);
  if (frx::grow_bytes(1000, 10) != 1000 || frx::grow_bytes(0, 1) != 256 || frx::grow_bytes(1024, 1025) != 1536) {
    printf("closed cases\n");
    bad = 1;
  }
  if (!bad) printf("policy_check ok\n");
  return bad;
}
