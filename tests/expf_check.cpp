// Host build of the router's expf restatement (mgpt_amd/csrc/glibc_expf.hpp),
// compared with the C library's expf over a range of float bit patterns.
// Usage: expf_check <first_bits_hex> <last_bits_hex>  -> prints mismatches.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include "../mgpt_amd/csrc/glibc_expf.hpp"

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  const uint32_t lo = (uint32_t)strtoul(argv[1], nullptr, 16);
  const uint32_t hi = (uint32_t)strtoul(argv[2], nullptr, 16);
  static const uint64_t T[32] = MGPT_EXP2_TABLE_INIT;
  unsigned long long mism = 0, n = 0;
  for (uint64_t u = lo; u <= hi; ++u) {
    uint32_t b = (uint32_t)u;
    float x;
    std::memcpy(&x, &b, 4);
    const float a = expf(x), c = mgpt_expf::expf_glibc(x, T);
    uint32_t ua, uc;
    std::memcpy(&ua, &a, 4);
    std::memcpy(&uc, &c, 4);
    if (ua != uc && !(std::isnan(a) && std::isnan(c))) {
      if (mism < 5) std::printf("mismatch x=%a expf=%a ours=%a\n", x, a, c);
      ++mism;
    }
    ++n;
  }
  std::printf("checked %llu mismatches %llu\n", n, mism);
  return mism ? 1 : 0;
}
