// Host harness for chunkkv_amd/csrc/cos_sin.hpp (the device kernels' cos/sin of fp32 angles).
//   cos_sin_sweep sweep LO HI THREADS : for every float bit pattern u in [LO, HI) and its negative,
//       compare cos_sin_fast with glibc's (float)cos/sin((double)x) bit for bit; print
//       "n <count> bad <count>" and up to 8 mismatches.
//   cos_sin_sweep eval : read float bit patterns (hex, one per line) from stdin, print
//       "<cos bits> <sin bits>" in hex per line (for the multiprecision spot check).
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "cos_sin.hpp"

static uint32_t bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

int main(int argc, char** argv) {
  if (argc >= 2 && std::strcmp(argv[1], "eval") == 0) {
    char line[64];
    while (std::fgets(line, sizeof line, stdin)) {
      const uint32_t u = (uint32_t)std::strtoul(line, nullptr, 16);
      float x, c, s;
      std::memcpy(&x, &u, 4);
      if (!ckv::cos_sin_fast(x, c, s)) {
        std::printf("none\n");
        continue;
      }
      std::printf("%08" PRIx32 " %08" PRIx32 "\n", bits(c), bits(s));
    }
    return 0;
  }
  if (argc != 5 || std::strcmp(argv[1], "sweep") != 0) return 2;
  const uint64_t lo = std::strtoull(argv[2], nullptr, 0), hi = std::strtoull(argv[3], nullptr, 0);
  const int nt = std::atoi(argv[4]);
  std::vector<uint64_t> n(nt), bad(nt);
  std::vector<std::vector<uint32_t>> first(nt);
  std::vector<std::thread> th;
  for (int t = 0; t < nt; ++t)
    th.emplace_back([&, t] {
      const uint64_t a = lo + (hi - lo) * t / nt, b = lo + (hi - lo) * (t + 1) / nt;
      for (uint64_t u = a; u < b; ++u)
        for (uint32_t sign : {0u, 0x80000000u}) {
          const uint32_t v = (uint32_t)u | sign;
          float x, c, s;
          std::memcpy(&x, &v, 4);
          ++n[t];
          if (!ckv::cos_sin_fast(x, c, s) || bits(c) != bits((float)std::cos((double)x)) ||
              bits(s) != bits((float)std::sin((double)x))) {
            ++bad[t];
            if (first[t].size() < 8) first[t].push_back(v);
          }
        }
    });
  uint64_t tn = 0, tb = 0;
  for (int t = 0; t < nt; ++t) {
    th[t].join();
    tn += n[t];
    tb += bad[t];
    for (uint32_t v : first[t]) std::printf("mismatch %08" PRIx32 "\n", v);
  }
  std::printf("n %" PRIu64 " bad %" PRIu64 "\n", tn, tb);
  return 0;
}
