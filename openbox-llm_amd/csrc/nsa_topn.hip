// Block importance + top-n selection (the block choice of NSAAttention,
// nsa_model.py:245-258 and :343-355).
//
// A workgroup of 4 waves takes 4 QPW consecutive queries of one (b, hkv); a
// wave holds the Q fragments of its QPW queries x P2 heads (P2 = 32 / QPW:
// the group padded to 16, 8 or 4 rows, a 32-row MFMA operand) and walks the
// pooled tokens the group's last query sees, 32 per tile, the tiles shared
// through LDS (direct global -> LDS loads, kImpStages deep).  Small groups
// (G <= 8, G <= 4) pack 4 or 8 queries into one tile instead of padding
// their heads to 16 rows:
//
//  1. S = Q K_cmp^T on 32x32 MFMAs (rows on M, tokens on N); p_cmp =
//     exp2(S * scale*log2e - lse_cmp*log2e) with lse_cmp from the compression
//     forward, tokens the query cannot see set to 0.
//  2. imp_cmp[q][i] = sum over the group's heads of p_cmp: a lane half holds
//     runs of consecutive rows of one query (8 heads of each of its 2 queries
//     when QPW = 2, whose two halves are then added; all 8 or 4 heads of its
//     own 2 or 4 queries when QPW = 4 or 8), summed in order (head chunks of
//     groups wider than 16 follow in chunk order), so every sum has a fixed
//     order.
//  3. every F tiles (and after the last) the tiles' tokens fold into the
//     selection blocks: imp_slc[j] += imp_cmp[i] * |span_i & block_j| / d,
//     tokens ascending, one lane per block for every query of the wave; F is
//     the most tiles whose blocks fit the wave's lanes.  The block sums live
//     in registers: lane L holds blocks L + 64 k (k < KPL) of each query, the
//     same layout the top-S phase reads (no LDS array per query, so long
//     sequences with thousands of blocks keep several workgroups per CU).  A
//     fold's 64 consecutive blocks fall in two register slots k, the same
//     for the whole wave, so only those two are updated.
//  4. per query: score = +inf for forced blocks, -FLT_MAX for blocks not yet
//     complete, else imp_slc; the order keys of the scores, KPL per lane in
//     registers (block lane + 64 k), give S picks, each the highest score by
//     a wave max and, among equal scores, the lowest block index by a wave
//     min.  With 8 or more keys per lane each lane first orders its 4 best
//     (ties by block index) and a pick pops the winning lane's head, the list
//     refilled from the lane's remaining keys when it runs empty; with fewer,
//     every pick rescans the lane's keys and zeroes the picked one.  Two
//     queries' picks interleave (two independent dependency chains) when
//     their keys fit the registers.
#include "nsa_launch.h"
#include "nsa_tile32.h"

namespace nsa {

constexpr int kImpFold = 8;               // tokens read per step of a block's fold
constexpr int kFoldTaps = 8;              // most tokens per block of the fixed-weight fold

// The fold's weights when a selection block is a whole number of strides
// (ls = R cd): token i = j R + r meets block j, for r = rlo .. rlo + n - 1,
// with the same weight w[r - rlo] = |[r cd, r cd + cl) & [0, ls)| / cd for
// every block j.  n = 0: other geometries (the fold computes each overlap).
struct FoldTaps {
  int n, rlo, R;
  float w[kFoldTaps];
};
constexpr int kImpFoldTiles = 8;          // most tiles per fold
constexpr int kImpStages = 3;             // K tiles in flight + 1

// last pooled token visible to t (-1: none)
__device__ __forceinline__ int imp_last_token(int t, int n_cmp, int cl, int cd) {
  if (t < cl - 1 || n_cmp <= 0) return -1;
  const int hi = (t - cl + 1) / cd;
  return hi < n_cmp - 1 ? hi : n_cmp - 1;
}

// x / 2^sh when sh >= 0 (x >= 0), else x / d
__device__ __forceinline__ int div_sh(int x, int d, int sh) { return sh >= 0 ? x >> sh : x / d; }

// Query of register run k (RUN consecutive registers) in lane half h: rows
// acc_elem(h, r) = 16 (r >> 3) + 8 h + (r & 7), query = row / P2.
template <int QPW>
__device__ __forceinline__ int imp_run_query(int k, int h) {
  if constexpr (QPW == 2) return k;                                // heads 8h..8h+7 of query k
  else if constexpr (QPW == 4) return 2 * k + h;                   // all 8 rows of query 2k+h
  else return 4 * (k >> 1) + 2 * h + (k & 1);                      // all 4 rows of query 4(k>>1)+2h+(k&1)
}

// Insert key x of slot k into a lane's list of its 4 best keys (m[0] >= m[1]
// >= ...; 0 = empty), when `take`.  Slots arrive in ascending order and only
// a strictly greater key moves ahead, so equal keys stay in slot order.
__device__ __forceinline__ void topn_list_insert(uint32_t (&m)[4], int (&c)[4], uint32_t x, int k, bool take) {
  const bool b0 = take && x > m[0], b1 = take && x > m[1], b2 = take && x > m[2], b3 = take && x > m[3];
  m[3] = b2 ? m[2] : (b3 ? x : m[3]);
  c[3] = b2 ? c[2] : (b3 ? k : c[3]);
  m[2] = b1 ? m[1] : (b2 ? x : m[2]);
  c[2] = b1 ? c[1] : (b2 ? k : c[2]);
  m[1] = b0 ? m[0] : (b1 ? x : m[1]);
  c[1] = b0 ? c[0] : (b1 ? k : c[1]);
  m[0] = b0 ? x : m[0];
  c[0] = b0 ? k : c[0];
}

// Waves per SIMD the register budget is cut to.  The walk's chain of
// dependent MFMAs, exponentials and per-tile barrier is latency-bound, so a
// third and fourth wave per SIMD pay even when the block sums they cost in
// registers (KPL per query) go to scratch: those are touched only by the
// fold (two slots a fold) and the picks.  16-bit inputs, two queries a wave,
// 512 to 2048 blocks (c5: 9.7 -> 7.2 ms); measured slower at five.
template <typename T, int KPL, int QPW>
constexpr int kImpWaves() {
  return sizeof(T) == 2 && QPW == 2 && KPL >= 8 && KPL <= 32 ? 4 : 1;
}

// LDS: K tiles [kImpStages][32][D] and per-wave token scratch [4][32 F][QPW]
// (the wave's queries' values of a token side by side).  cd_sh / ls_sh: log2
// of cd / ls when they are powers of two, else -1 (the block fold then
// divides); rcd = 1 / cd scales the overlap weights; fold_tiles: F above
// (1 .. kImpFoldTiles).  KPL: blocks per lane (n_slc <= 64 * KPL).
template <typename T, int D, int KPL, int QPW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kImpWaves<T, KPL, QPW>()))) void k_imp_topn(const T* __restrict__ q, const T* __restrict__ kc,
                                                  const float* __restrict__ lse, int32_t* __restrict__ out_idx,
                                                  float* __restrict__ scores, int Hq, int Hkv, int T_, int n_cmp,
                                                  int n_slc, int S, int cl, int cd, int ls, int force_init,
                                                  int n_local, int nqb, int cd_sh, int ls_sh, int fold_tiles, float rcd, float sl2,
                                                  const FoldTaps taps) {
  using C = Tile32<T, D>;
  constexpr int NST = kImpStages;
  constexpr int P2 = 32 / QPW;              // rows per query
  constexpr int RUN = QPW == 8 ? 4 : 8;     // consecutive registers of one query in a lane half
  constexpr int NRUN = 16 / RUN;            // query partials per lane
  constexpr int QPB = 4 * QPW;              // queries per workgroup
  static_assert(QPW == 2 || QPW == 4 || QPW == 8, "2, 4 or 8 queries per wave");
  extern __shared__ __align__(16) char smem[];
  T* sK = reinterpret_cast<T*>(smem);                                   // [NST][ROW_ELEMS]
  float* stok = reinterpret_cast<float*>(sK + NST * C::ROW_ELEMS);      // [4][32 F][QPW]
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // long rows first: workgroups go out round-robin, the latest queries first
  const int qb = nqb - 1 - (int)(blockIdx.x % nqb);
  const int bh = (int)(blockIdx.x / nqb);
  const int b = bh / Hkv, hkv = bh % Hkv;
  const int G = Hq / Hkv, NHC = (G + 15) / 16;   // NHC > 1 only with QPW == 2
  const int t0 = qb * QPB;
  const int tq0 = t0 + QPW * w;   // this wave's queries tq0 .. tq0 + QPW - 1
  const int tlast = t0 + QPB - 1 < T_ - 1 ? t0 + QPB - 1 : T_ - 1;
  const int hi_wg = imp_last_token(tlast, n_cmp, cl, cd);
  const int ntile = hi_wg < 0 ? 0 : hi_wg / 32 + 1;
  int hi_q[QPW];
#pragma unroll
  for (int i = 0; i < QPW; ++i) hi_q[i] = tq0 + i < T_ ? imp_last_token(tq0 + i, n_cmp, cl, cd) : -1;
  // the last visible token of each register run's query (runs of lane half h)
  int hi_run[NRUN];
#pragma unroll
  for (int k = 0; k < NRUN; ++k) hi_run[k] = h ? hi_q[imp_run_query<QPW>(k, 1)] : hi_q[imp_run_query<QPW>(k, 0)];

  float bsum[QPW][KPL];   // block sums of blocks lane + 64 k, every query of the wave
#pragma unroll
  for (int i = 0; i < QPW; ++i)
#pragma unroll
    for (int k = 0; k < KPL; ++k) bsum[i][k] = 0.0f;
  const T* kbase = kc + (int64_t)bh * n_cmp * D;
  RowTileDma<T, D, 256, true> kdma;
  kdma.init(tid);
  auto load_tile = [&](int kt) { kdma.request(sK + (kt % NST) * C::ROW_ELEMS, kbase, kt * 32, n_cmp, tid); };

  // this lane's 16 rows: e = acc_elem(h, r) -> query e / P2, head e % P2
  float* my_tok = stok + w * 32 * kImpFoldTiles * QPW;
  Frag<T> qf[C::KS];
  float lse2[16];
  auto load_rows = [&](int hc) {
    const int row = perm32(n);            // A operand row this lane supplies
    const int hd = hc * 16 + row % P2;
    const int hs = hd < G ? hd : G - 1;
    int tq = tq0 + row / P2;
    tq = tq < T_ ? tq : T_ - 1;
    const T* qrow = q + (((int64_t)b * Hq + hkv * G + hs) * T_ + tq) * D;
#pragma unroll
    for (int s = 0; s < C::KS; ++s) qf[s].load(qrow + 16 * s + 8 * h);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int e = acc_elem(h, r);
      const int he = hc * 16 + e % P2;
      int te = tq0 + e / P2;
      const bool ok = he < G && te < T_;
      te = te < T_ ? te : T_ - 1;
      // absent rows (padding heads, queries past T) get p = 0
      lse2[r] = ok ? lse[((int64_t)b * Hq + hkv * G + he) * T_ + te] * kLog2e : __builtin_inff();
    }
    // complete these loads here: the walk's own loads are asm the compiler
    // does not see, so a wait it placed later (e.g. before the first MFMA)
    // would also drain the K tiles in flight
#pragma unroll
    for (int s = 0; s < C::KS; ++s) settle(qf[s]);
#pragma unroll
    for (int r = 0; r < 16; ++r) asm volatile("" : "+v"(lse2[r]));
  };
  if (NHC == 1) load_rows(0);
  key_pipeline<NST, dma_uniform_loads<256, C::ROW_CHUNKS>()>(ntile, load_tile, [&](int kt) {
    const T* tile = sK + (kt % NST) * C::ROW_ELEMS;
    const int tok = kt * 32 + n;
    float* slot = my_tok + ((kt % fold_tiles) * 32 + n) * QPW;
    for (int hc = 0; hc < NHC; ++hc) {
      if (NHC > 1) load_rows(hc);   // groups wider than 16 heads: one chunk at a time
      f32x16 sacc = zero16();
#pragma unroll
      for (int s = 0; s < C::KS; ++s) {
        Frag<T> kf;
        lds_nrow_frag<T, D>(kf, tile, n, h, s);
        mma32(sacc, qf[s], kf);
      }
      float part[NRUN];
#pragma unroll
      for (int k = 0; k < NRUN; ++k) {
        float acc = fast_exp2(sacc[RUN * k] * sl2 - lse2[RUN * k]);
#pragma unroll
        for (int j = 1; j < RUN; ++j) acc += fast_exp2(sacc[RUN * k + j] * sl2 - lse2[RUN * k + j]);
        part[k] = tok <= hi_run[k] ? acc : 0.0f;   // tokens the query cannot see
      }
      if constexpr (QPW == 2) {
        // heads 8h .. 8h+7 of each query are in lane half h: the half swap
        // gives both halves part(half 0) and part(half 1); their sum is the
        // same in every lane, and lane half 0 keeps it
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(part[k]), __float_as_uint(part[k]),
                                                           false, false);
          part[k] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        if (h == 0) {
          float2* sl2p = reinterpret_cast<float2*>(slot);
          if (hc == 0) {
            *sl2p = make_float2(part[0], part[1]);
          } else {
            const float2 o = *sl2p;
            *sl2p = make_float2(o.x + part[0], o.y + part[1]);
          }
        }
      } else if constexpr (QPW == 4) {
        // lane half h holds queries h and 2 + h whole
        slot[h] = part[0];
        slot[2 + h] = part[1];
      } else {
        // lane half h holds queries 2h, 2h + 1, 4 + 2h, 5 + 2h whole
        *reinterpret_cast<float2*>(slot + 2 * h) = make_float2(part[0], part[1]);
        *reinterpret_cast<float2*>(slot + 4 + 2 * h) = make_float2(part[2], part[3]);
      }
    }
    if (kt % fold_tiles != fold_tiles - 1 && kt != ntile - 1) return;
    wave_fence();
    // fold the last tiles' tokens into the blocks they overlap, tokens
    // ascending; the blocks touched (at most 64: fold_tiles is chosen so)
    // go one to a lane, block j to lane j % 64 (its register slot j / 64);
    // the block's tokens are read kImpFold at a time so their LDS reads
    // overlap
    const int i0 = (kt - kt % fold_tiles) * 32;
    const int i1 = kt * 32 + 31 < n_cmp - 1 ? kt * 32 + 31 : n_cmp - 1;
    const int jlo = div_sh(i0 * cd, ls, ls_sh);
    int jhi = div_sh(i1 * cd + cl - 1, ls, ls_sh);
    jhi = jhi < n_slc - 1 ? jhi : n_slc - 1;
    const int j = jlo + ((lane - jlo) & (kWave - 1));
    if (j <= jhi) {
      const int kj = j / kWave;
      // tokens whose span [i*cd, i*cd+cl) meets [j*ls, (j+1)*ls)
      int a_i = j * ls - cl + 1 <= 0 ? 0 : div_sh(j * ls - cl + 1 + cd - 1, cd, cd_sh);
      int b_i = div_sh((j + 1) * ls - 1, cd, cd_sh);
      a_i = a_i > i0 ? a_i : i0;
      b_i = b_i < i1 ? b_i : i1;
      const float* tq = my_tok - i0 * QPW;
      float sq[QPW];   // this fold's share of the block's sums, every query
#pragma unroll
      for (int u = 0; u < QPW; ++u) sq[u] = 0.0f;
      if (taps.n > 0) {
        // the same tokens a_i .. b_i in the same order with the same
        // weights, without the per-token overlap arithmetic
        const int ib0 = j * taps.R + taps.rlo;
        float v[kFoldTaps][QPW];
#pragma unroll
        for (int x = 0; x < kFoldTaps; ++x) {
          const int i = ib0 + x;
          const float* src = tq + (i >= a_i && i <= b_i ? i : a_i) * QPW;
#pragma unroll
          for (int u = 0; u < QPW; u += 2) {
            const float2 t2 = *reinterpret_cast<const float2*>(src + u);
            v[x][u] = t2.x;
            v[x][u + 1] = t2.y;
          }
        }
#pragma unroll
        for (int x = 0; x < kFoldTaps; ++x) {
          const int i = ib0 + x;
          if (x < taps.n && i >= a_i && i <= b_i) {
#pragma unroll
            for (int u = 0; u < QPW; ++u) sq[u] += v[x][u] * taps.w[x];
          }
        }
      } else
      for (int ib = a_i; ib <= b_i; ib += kImpFold) {
        float v[kImpFold][QPW];
#pragma unroll
        for (int x = 0; x < kImpFold; ++x) {
          const float* src = tq + (ib + x <= b_i ? ib + x : b_i) * QPW;
#pragma unroll
          for (int u = 0; u < QPW; u += 2) {
            const float2 t2 = *reinterpret_cast<const float2*>(src + u);
            v[x][u] = t2.x;
            v[x][u + 1] = t2.y;
          }
        }
#pragma unroll
        for (int x = 0; x < kImpFold; ++x) {
          const int i = ib + x;
          const int a = i * cd > j * ls ? i * cd : j * ls;
          const int e = i * cd + cl < (j + 1) * ls ? i * cd + cl : (j + 1) * ls;
          if (i <= b_i && e > a) {
            const float wgt = (float)(e - a) * rcd;
#pragma unroll
            for (int u = 0; u < QPW; ++u) sq[u] += v[x][u] * wgt;
          }
        }
      }
      // the fold's blocks jlo .. jlo + 63 sit in register slots kj0 and
      // kj0 + 1 of every lane (kj0 is the same for the whole wave): only
      // those two slots are updated
      const int kj0 = jlo / kWave;
#pragma unroll
      for (int k = 0; k < KPL; ++k) {
        if (k == kj0 || k == kj0 + 1) {
#pragma unroll
          for (int u = 0; u < QPW; ++u) bsum[u][k] += kj == k ? sq[u] : 0.0f;
        }
      }
    }
    wave_fence();
  });

  // per query of this wave: scores, masking and forcing, then top-S
  constexpr int QIL = KPL <= 32 ? 2 : 1;   // queries whose picks interleave
#pragma unroll
  for (int q0 = 0; q0 < QPW; q0 += QIL) {
    uint32_t key[QIL][KPL];   // order key of block lane + 64 k; 0 once picked and for absent blocks
    bool live[QIL];
    int32_t* orow[QIL];
    int pick[QIL];
#pragma unroll
    for (int u = 0; u < QIL; ++u) {
      const int t = tq0 + q0 + u;
      live[u] = t < T_;
      const int64_t r = (int64_t)bh * T_ + t;
      orow[u] = out_idx + r * S;
      pick[u] = 0;
      const int tb = t / ls;
#pragma unroll
      for (int k = 0; k < KPL; ++k) {
        const int j = lane + kWave * k;
        key[u][k] = 0;
        if (live[u] && j < n_slc) {
          const float s = bsum[q0 + u][k];
          if (scores != nullptr) scores[r * n_slc + j] = s;
          const bool valid = (j + 1) * ls - 1 <= t;
          const bool forced = (force_init && j == 0) || (j <= tb && j > tb - n_local);
          key[u][k] = order_key(forced ? __builtin_inff() : (valid ? s : -3.4028234663852886e38f));
        }
      }
    }
    if constexpr (KPL >= 8) {
      // each lane keeps its 4 best keys in order (key descending, slot
      // ascending among equal keys); a pick takes the wave's best list head
      // and pops it from its lane's list.  A lane's popped keys are always a
      // prefix of its order, so a list that runs empty is refilled with the
      // next 4 after the last popped one.
      uint32_t lm[QIL][4];
      int lc[QIL][4];
      uint32_t last_m[QIL];
      int last_c[QIL];
#pragma unroll
      for (int u = 0; u < QIL; ++u) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lm[u][i] = 0u;
          lc[u][i] = KPL;
        }
        last_m[u] = 0xFFFFFFFFu;
        last_c[u] = -1;
#pragma unroll
        for (int k = 0; k < KPL; ++k) topn_list_insert(lm[u], lc[u], key[u][k], k, true);
      }
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int u = 0; u < QIL; ++u) {
          const uint32_t top = wave_reduce_u32<true>(lm[u][0]);
          const int jw = (int)__builtin_amdgcn_readfirstlane(
              (int)wave_reduce_u32<false>(lm[u][0] == top ? (uint32_t)(lane + kWave * lc[u][0]) : 0xFFFFFFFFu));
          pick[u] = lane == (s & (kWave - 1)) ? jw : pick[u];
          const bool own = lane == (jw & (kWave - 1));
          last_m[u] = own ? lm[u][0] : last_m[u];
          last_c[u] = own ? lc[u][0] : last_c[u];
#pragma unroll
          for (int i = 0; i < 3; ++i) {
            lm[u][i] = own ? lm[u][i + 1] : lm[u][i];
            lc[u][i] = own ? lc[u][i + 1] : lc[u][i];
          }
          lm[u][3] = own ? 0u : lm[u][3];
          lc[u][3] = own ? KPL : lc[u][3];
          const bool refill = own && lm[u][0] == 0u;
          if (__builtin_amdgcn_ballot_w64(refill) != 0) {   // wave-uniform
#pragma unroll
            for (int k = 0; k < KPL; ++k) {
              const uint32_t x = key[u][k];
              const bool after = x < last_m[u] || (x == last_m[u] && k > last_c[u]);
              topn_list_insert(lm[u], lc[u], x, k, refill && after);
            }
          }
        }
        if ((s & (kWave - 1)) == kWave - 1 || s == S - 1) {
#pragma unroll
          for (int u = 0; u < QIL; ++u)
            if (live[u] && lane <= (s & (kWave - 1))) orow[u][(s & ~(kWave - 1)) + lane] = pick[u];
        }
      }
    } else {
      // few keys per lane: scan them at every pick
      for (int s = 0; s < S; ++s) {
#pragma unroll
        for (int u = 0; u < QIL; ++u) {
          uint32_t m = key[u][0];
#pragma unroll
          for (int k = 1; k < KPL; ++k) m = key[u][k] > m ? key[u][k] : m;
          int kb = 0;   // this lane's lowest k holding m
#pragma unroll
          for (int k = KPL - 1; k > 0; --k) kb = key[u][k] == m ? k : kb;
          kb = key[u][0] == m ? 0 : kb;
          const uint32_t top = wave_reduce_u32<true>(m);
          const int jw = (int)__builtin_amdgcn_readfirstlane(
              (int)wave_reduce_u32<false>(m == top ? (uint32_t)(lane + kWave * kb) : 0xFFFFFFFFu));
          pick[u] = lane == (s & (kWave - 1)) ? jw : pick[u];
          const bool own = lane == (jw & (kWave - 1));
#pragma unroll
          for (int k = 0; k < KPL; ++k) key[u][k] = own && k == jw / kWave ? 0u : key[u][k];
        }
        if ((s & (kWave - 1)) == kWave - 1 || s == S - 1) {
#pragma unroll
          for (int u = 0; u < QIL; ++u)
            if (live[u] && lane <= (s & (kWave - 1))) orow[u][(s & ~(kWave - 1)) + lane] = pick[u];
        }
      }
    }
  }
}

}  // namespace nsa

using namespace nsa;

extern "C" {

int nsa_importance_topn(const void* q, const void* k_cmp, const float* lse_cmp, int32_t* block_idx, float* scores,
                        int B, int Hq, int Hkv, int T, int n_cmp, int D, int cmp_block, int cmp_stride,
                        int sel_block, int n_sel, int force_init, int n_local, int dtype, void* stream) {
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && n_cmp >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(cmp_block >= 1 && cmp_stride >= 1 && sel_block >= 1 && n_sel >= 0 && n_local >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  const int n_slc = T / sel_block;
  const int S = n_sel < n_slc ? n_sel : n_slc;
  NSA_CHECK(n_slc <= 64 * 64, NSA_ERR_SHAPE);
  if (T == 0 || n_slc == 0) return NSA_OK;
  // blocks per lane (registers: block sums, then order keys)
  const int kpl = n_slc <= 64 * 2 ? 2 : n_slc <= 64 * 8 ? 8 : n_slc <= 64 * 16 ? 16 : n_slc <= 64 * 32 ? 32 : 64;
  // queries per wave: the group's heads padded to 16, 8 or 4 rows of the
  // 32-row tile, while the block sums (queries x blocks per lane) fit 64
  // registers (128 at two queries)
  const int G = Hq / Hkv;
  int qpw = G > 8 ? 2 : G > 4 ? 4 : 8;
  while (qpw > 2 && qpw * kpl > 64) qpw /= 2;
  const size_t ksz = (dtype == NSA_BF16 ? 2 : 4) * (size_t)kImpStages * 32 * D;
  const size_t lds = ksz + sizeof(float) * ((size_t)4 * qpw * 32 * kImpFoldTiles);
  NSA_CHECK(lds <= 160 * 1024, NSA_ERR_SHAPE);
  const int nqb = (T + 4 * qpw - 1) / (4 * qpw);
  const int64_t grid = (int64_t)B * Hkv * nqb;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  const float sl2 = (1.0f / sqrtf((float)D)) * kLog2e;
  const int cd_sh = (cmp_stride & (cmp_stride - 1)) == 0 ? __builtin_ctz(cmp_stride) : -1;
  const int ls_sh = (sel_block & (sel_block - 1)) == 0 ? __builtin_ctz(sel_block) : -1;
  const float rcd = 1.0f / (float)cmp_stride;
  // tiles per fold: the most (up to kImpFoldTiles) whose tokens' blocks fit
  // the wave's lanes
  FoldTaps taps{};
  if (sel_block % cmp_stride == 0) {
    const int rlo = -((cmp_block - 1) / cmp_stride), rhi = (sel_block - 1) / cmp_stride;
    if (rhi - rlo + 1 <= kFoldTaps) {
      taps.n = rhi - rlo + 1;
      taps.rlo = rlo;
      taps.R = sel_block / cmp_stride;
      for (int x = 0; x < taps.n; ++x) {
        const int p0 = (rlo + x) * cmp_stride;   // the token's span relative to the block start
        const int a = p0 > 0 ? p0 : 0;
        const int e = p0 + cmp_block < sel_block ? p0 + cmp_block : sel_block;
        taps.w[x] = (float)(e - a) * rcd;
      }
    }
  }
  int fold_tiles = 1;
  for (int f = 2; f <= kImpFoldTiles; ++f) {
    const int64_t span = (int64_t)(32 * f - 1) * cmp_stride + cmp_block;   // positions the tokens cover
    if ((span - 1) / sel_block + 2 <= 64) fold_tiles = f;
  }
  hipStream_t s = (hipStream_t)stream;
  // more than 64 KB of dynamic LDS must be allowed per kernel
  auto launch = [&](auto kern, auto qp, auto kp) -> int {
    if (lds > 65536 && hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
                           hipSuccess)
      return NSA_ERR_LAUNCH;
    kern<<<(unsigned)grid, 256, lds, s>>>(qp, kp, lse_cmp, block_idx, scores, Hq, Hkv, T, n_cmp, n_slc, S,
                                          cmp_block, cmp_stride, sel_block, force_init, n_local, nqb, cd_sh, ls_sh,
                                          fold_tiles, rcd, sl2, taps);
    return NSA_OK;
  };
  int rc = NSA_ERR_SHAPE;
#define NSA_TOPN_KQ(DD, KK, QQ)                                                                        \
  if (kpl == KK && qpw == QQ)                                                                          \
    rc = dtype == NSA_BF16 ? launch(k_imp_topn<bf16, DD, KK, QQ>, (const bf16*)q, (const bf16*)k_cmp) \
                           : launch(k_imp_topn<float, DD, KK, QQ>, (const float*)q, (const float*)k_cmp);
#define NSA_TOPN_CASE(DD)                                                 \
  case DD:                                                                \
    NSA_TOPN_KQ(DD, 2, 2) NSA_TOPN_KQ(DD, 2, 4) NSA_TOPN_KQ(DD, 2, 8)     \
    NSA_TOPN_KQ(DD, 8, 2) NSA_TOPN_KQ(DD, 8, 4) NSA_TOPN_KQ(DD, 8, 8)     \
    NSA_TOPN_KQ(DD, 16, 2) NSA_TOPN_KQ(DD, 16, 4)                         \
    NSA_TOPN_KQ(DD, 32, 2)                                                \
    NSA_TOPN_KQ(DD, 64, 2)                                                \
    break;
  switch (D) {
    NSA_TOPN_CASE(16)
    NSA_TOPN_CASE(32)
    NSA_TOPN_CASE(64)
    NSA_TOPN_CASE(128)
    default:
      break;
  }
#undef NSA_TOPN_CASE
#undef NSA_TOPN_KQ
  if (rc != NSA_OK) return rc;
  return nsa_launch_status();
}

}  // extern "C"
