// Host-side check of the row clamp of a [32][D] row-tile request (tile_rows
// in nsa_tile32.h, used by RowTileDma::request).  Lane row r of a tile from
// r0 reads byte base(tile_rows.base) + off(r) - (r > last ? (r - last) rows : 0)
// with unsigned 32-bit offsets.  For every start r0, also at and past the end
// of the source, every row's address must fall inside the source and equal
// row min(r0 + r, nrows - 1).  The earlier form (base r0, last = nrows - 1 -
// r0) is evaluated beside it: for r0 >= nrows its offsets wrap, the
// out-of-bounds read of a top-n variant whose last tile started past the
// pooled keys.
#include <cstdint>
#include <cstdio>

#include "nsa_tile32.h"

int main() {
  const int D = 128;
  const uint32_t rb = D * 2;   // bf16 rows
  int bad = 0, wrapped_old = 0, cases = 0;
  for (int nrows = 1; nrows < 140; nrows += 3)
    for (int r0 = 0; r0 < nrows + 40; ++r0) {
      const nsa::TileRows tr = nsa::tile_rows(r0, nrows);
      for (int r = 0; r < 32; ++r)
        for (uint32_t c = 0; c < rb; c += 64) {
          uint32_t o = (uint32_t)r * rb + c;
          if (tr.last < 31 && r > tr.last) o -= (uint32_t)(r - tr.last) * rb;
          const uint64_t a = (uint64_t)tr.base * rb + o;
          const int want = r0 + r < nrows ? r0 + r : nrows - 1;
          if (a != (uint64_t)want * rb + c || a >= (uint64_t)nrows * rb) ++bad;
          const int last_old = nrows - 1 - r0;
          uint32_t oo = (uint32_t)r * rb + c;
          if (last_old < 31 && r > last_old) oo -= (uint32_t)(r - last_old) * rb;
          if ((uint64_t)r0 * rb + oo >= (uint64_t)nrows * rb) ++wrapped_old;
          ++cases;
        }
    }
  std::printf("cases %d, wrong %d, out-of-range addresses of the earlier form %d\n", cases, bad, wrapped_old);
  return bad == 0 && wrapped_old > 0 ? 0 : 1;
}
