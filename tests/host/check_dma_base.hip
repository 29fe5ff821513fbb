// Host-side check of the address arithmetic of the SGPR-base DMA helper
// (lds_dma16_sbase in nsa_tile32.h): a 64-bit device address is split into
// two 32-bit halves, each passed through readfirstlane (which returns int),
// and joined again.  Bases whose low half has bit 31 set must come back
// unchanged; the earlier form, which widened the int low half directly,
// sign-extended it and corrupted the high half.
#include <cstdint>
#include <cstdio>

#include "nsa_tile32.h"

static uint64_t sign_extending_join(int lo, int hi) {   // the faulty form, for contrast
  return ((uint64_t)(uint32_t)hi << 32) | (uint64_t)(int64_t)lo;
}

int main() {
  const uint64_t bases[] = {0x00007ffe80001000ull, 0x00007fffffffff00ull, 0x0000000080000000ull,
                            0x00007ffe00001000ull, 0x0000600000000000ull, 0x00007ffefffffff0ull};
  int bad = 0, caught = 0;
  for (uint64_t b : bases) {
    const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
    const uint64_t got = nsa::u64_from_halves(lo, hi);
    if (got != b) {
      std::printf("FAIL %016llx -> %016llx\n", (unsigned long long)b, (unsigned long long)got);
      ++bad;
    }
    if ((b & 0x80000000ull) && sign_extending_join(lo, hi) != b) ++caught;
  }
  std::printf("bases %zu, wrong %d, bit-31 bases the sign-extending join corrupts %d\n",
              sizeof(bases) / sizeof(bases[0]), bad, caught);
  return bad == 0 && caught == 4 ? 0 : 1;
}
