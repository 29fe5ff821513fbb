// Host-side check of the flat-row visibility of the range dK/dV (groups of
// G < 16 heads: row R of a group is query R / G; flat_rows_seeing and
// flat_tile_needs_mask in nsa_tile32.h).  Against brute force over the 32
// rows of a tile: the row mask of a key, and that a tile declared free of
// the per-element test has every present row seeing all 32 keys of the wave.
#include <cstdint>
#include <cstdio>

#include "nsa_tile32.h"

static bool sees(int key, int t, int window, int cl, int cd) {
  return window > 0 ? (key <= t && t < key + window) : (key * cd + cl - 1 <= t);
}

int main() {
  const int windows[] = {0, 1, 3, 32, 512};
  const int geo[][2] = {{32, 16}, {16, 16}, {48, 32}, {1, 1}};
  long cases = 0, bad_bits = 0, bad_mask = 0, skipped_tiles = 0;
  for (int G = 1; G < 16; ++G)
    for (int window : windows)
      for (const auto& cg : geo) {
        const int cl = cg[0], cd = cg[1];
        for (int R0 = 0; R0 < 2600; R0 += 13) {
          const int rhi = R0 + 20 + (R0 % 17);   // the last present row, sometimes inside the tile
          for (int kw = 0; kw < 700; kw += 29) {
            bool all_seen = true;
            for (int key = kw; key < kw + 32; ++key) {
              uint32_t want = 0;
              for (int r = 0; r < 32; ++r) {
                const int t = (R0 + r) / G;
                const bool s = sees(key, t, window, cl, cd);
                if (s) want |= 1u << r;
                if (R0 + r <= rhi && !s) all_seen = false;
              }
              if (nsa::flat_rows_seeing(key, R0, G, window, cl, cd) != want) ++bad_bits;
              ++cases;
            }
            const bool need = nsa::flat_tile_needs_mask(kw, R0, rhi, G, window, cl, cd);
            if (!need) {
              ++skipped_tiles;
              if (!all_seen) ++bad_mask;
            }
          }
        }
      }
  std::printf("keys %ld, wrong row masks %ld, tiles without the test %ld, of which wrongly %ld\n", cases,
              bad_bits, skipped_tiles, bad_mask);
  return bad_bits == 0 && bad_mask == 0 && skipped_tiles > 0 ? 0 : 1;
}
