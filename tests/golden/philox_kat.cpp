// Host program: prints Philox4x32-10 known-answer vectors from rocRAND's header
// (the engine's ten_rounds), as JSON, for tests/golden/philox_kat.json.
#include <hip/hip_runtime.h>
#include <rocrand/rocrand_philox4x32_10.h>
#include <cstdio>

struct Exposed : rocrand_device::philox4x32_10_engine {
  uint4 rounds(uint4 c, uint2 k) { return ten_rounds(c, k); }
};

int main() {
  const unsigned cases[][6] = {
      {0u, 0u, 0u, 0u, 0u, 0u},
      {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu},
      {0x243f6a88u, 0x85a308d3u, 0x13198a2eu, 0x03707344u, 0xa4093822u, 0x299f31d0u},
      {7u, 123456u, 0u, 1u, 0xdeadbeefu, 0x01234567u},
      {63u, 5u, 0u, 0u, 42u, 0u},
  };
  Exposed e;
  std::printf("[");
  for (int i = 0; i < 5; ++i) {
    const unsigned* c = cases[i];
    uint4 r = e.rounds(uint4{c[0], c[1], c[2], c[3]}, uint2{c[4], c[5]});
    std::printf("%s{\"ctr\":[%u,%u,%u,%u],\"key\":[%u,%u],\"out\":[%u,%u,%u,%u]}",
                i ? "," : "", c[0], c[1], c[2], c[3], c[4], c[5], r.x, r.y, r.z, r.w);
  }
  std::printf("]\n");
  return 0;
}
