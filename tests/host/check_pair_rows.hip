// Host-side check of the row addressing of a selection tile's two queries
// (pair_rows in nsa_tile32.h, used by the dK/dV and forward tile requests).
// A request reads query A's rows at base(t0) + per-lane offset + dA and query
// B's at base(t0) + per-lane offset + dB, all offsets unsigned 32-bit.  For
// every order of (tA, tB), and tB = -1 (none), each lane's byte address must
// land on its own query's row.  The earlier form took both offsets from tA,
// so a CSR whose entries do not ascend (tB < tA) wrapped query B's offset to
// about 4 GB past the base -- the out-of-bounds read of a timing probe that
// fed such a CSR.
#include <cstdint>
#include <cstdio>

#include "nsa_tile32.h"

int main() {
  const int T = 300;
  const uint32_t rb = 16 * 128 * 2;   // one packed query: 16 heads x 128 d, bf16
  int bad = 0, wrapped_old = 0, cases = 0;
  for (int tA = 0; tA < T; tA += 7)
    for (int tB = -1; tB < T; tB += 5) {
      const nsa::PairRows p = nsa::pair_rows(tA, tB, rb);
      const int tb = tB >= 0 ? tB : tA;
      for (uint32_t lane_off = 0; lane_off < rb; lane_off += 1024) {
        const uint64_t a = (uint64_t)p.t0 * rb + (uint32_t)(lane_off + p.dA);
        const uint64_t b = (uint64_t)p.t0 * rb + (uint32_t)(lane_off + p.dB);
        if (a != (uint64_t)tA * rb + lane_off || b != (uint64_t)tb * rb + lane_off) ++bad;
        // the earlier form: base at tA, query B at (uint32)(tb - tA) * rb
        const uint64_t b_old = (uint64_t)tA * rb + (uint32_t)(lane_off + (uint32_t)(tb - tA) * rb);
        if (b_old >= (uint64_t)T * rb) ++wrapped_old;
        ++cases;
      }
    }
  std::printf("cases %d, wrong %d, out-of-range addresses of the earlier form %d\n", cases, bad, wrapped_old);
  return bad == 0 && wrapped_old > 0 ? 0 : 1;
}
