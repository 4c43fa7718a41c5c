// Copies of many sizes through sy::CopyPool (simdyolo_amd/csrc/host_copy.h):
// every byte arrives, whatever the split between the pool's threads (sizes
// include those whose floor share is a page multiple with a remainder).
#include <cstdio>
#include <random>
#include <vector>

#include "host_copy.h"

int main() {
  std::mt19937_64 rng(7);
  for (int workers : {0, 3, 5}) {
    sy::CopyPool pool(workers);
    for (int it = 0; it < 300; ++it) {
      size_t n = (rng() % (12u << 20)) + 1;
      if (it % 3 == 0) n = (size_t)(workers + 1) * 4096 * (1 + rng() % 300) + 4 * (1 + rng() % 5);
      std::vector<unsigned char> a(n), b(n, 0);
      for (size_t k = 0; k < n; ++k) a[k] = (unsigned char)(k * 131 + it);
      pool.copy(b.data(), a.data(), n);
      if (a != b) {
        std::printf("FAIL workers %d bytes %zu\n", workers, n);
        return 1;
      }
      std::vector<unsigned char> c(n, 1);
      pool.touch(c.data(), n);
      for (size_t k = 0; k < n; k += 4096)
        if (c[k] != 0) {
          std::printf("FAIL touch workers %d bytes %zu page %zu\n", workers, n, k / 4096);
          return 1;
        }
    }
  }
  std::printf("ok\n");
  return 0;
}
