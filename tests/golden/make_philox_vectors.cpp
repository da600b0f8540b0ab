// Writes Philox4x32-10 known-answer vectors from rocRAND's engine (MIT,
// /opt/rocm/include/rocrand/rocrand_philox4x32_10.h), an implementation
// independent of this repository's, to pin the oracle and the kernel.
// Build and run (host only):
//   hipcc -O1 tests/golden/make_philox_vectors.cpp -o /tmp/mk && /tmp/mk > tests/golden/philox_rocrand.json
#include <rocrand/rocrand_philox4x32_10.h>
#include <cstdio>
#include <cstdint>

// ten_rounds() is protected: a subclass exposes it.
struct Engine : rocrand_device::philox4x32_10_engine {
  uint4 rounds(uint4 c, uint2 k) { return ten_rounds(c, k); }
};

int main() {
  Engine eng;
  const uint32_t cases[][6] = {
      {0u, 0u, 0u, 0u, 0u, 0u},
      {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu},
      {0x243f6a88u, 0x85a308d3u, 0x13198a2eu, 0x03707344u, 0xa4093822u, 0x299f31d0u},
      {1u, 0u, 0u, 0u, 0u, 0u},
      {0u, 0u, 0u, 0u, 1u, 0u},
      {7u, 3u, 0u, 0u, 0x12345678u, 0x9abcdef0u},
      {255u, 0x00010000u, 0u, 0u, 0xdeadbeefu, 0x00c0ffeeu},
  };
  std::printf("[\n");
  const int n = sizeof(cases) / sizeof(cases[0]);
  for (int i = 0; i < n; ++i) {
    uint4 ctr{cases[i][0], cases[i][1], cases[i][2], cases[i][3]};
    uint2 key{cases[i][4], cases[i][5]};
    uint4 r = eng.rounds(ctr, key);
    std::printf("  {\"counter\": [%u, %u, %u, %u], \"key\": [%u, %u], \"out\": [%u, %u, %u, %u]}%s\n",
                ctr.x, ctr.y, ctr.z, ctr.w, key.x, key.y, r.x, r.y, r.z, r.w, i + 1 < n ? "," : "");
  }
  std::printf("]\n");
  return 0;
}
