// Key-side NSA backward: dK/dV of the range branches (window, compression)
// and of the selection branch (block-outer over the block -> query CSR),
// LDS-tiled on 32x32 MFMAs.
//
// A wave owns 32 keys: their K and V fragments stay in registers and their
// dK^T / dV^T accumulate in registers for the whole walk.  The queries that
// see those keys stream through LDS two at a time (32 rows = two queries x 16
// heads of a head chunk): row tiles of Q and dO, their transposed copies
// (direct global -> LDS loads, double-buffered) and per-row statistics
// c = lse*log2(e) - log2(rowscale) (+inf for rows that do not exist) and
// delta, shared by the workgroup's waves.
//   S = Q K^T, dP = dO V^T                     (rows on M, keys on N)
//   P = exp2(S*scale*log2(e) - c), dS = P (dP - delta)
//   dV^T += dO^T P,  dK^T += Q^T dS             (P / dS straight from the accumulators)
// Query rows of Q / dO are read through perm32 so the S / dP accumulators
// line up with the operand slots of the second pair of contractions.  Tiles
// whose two queries see all 32 keys of a wave skip the per-element mask.
//
//   * window      : a workgroup owns 32*NW keys and walks queries [k0, k0 + 32 NW + w - 2];
//                   one writer per key, plain stores.
//   * compression : same, over query chunks of kCmpChunk (grid.y); chunks merge with
//                   float atomics.
//   * selection   : work items (block, chunk of its CSR query list) built by
//                   k_sel_items; a persistent grid drains them; chunks merge with atomics.
#include "nsa_launch.h"
#include "nsa_items.h"
#include "nsa_tile32.h"

namespace nsa {

template <typename T, int D> struct KvStage {
  using C = Tile32<T, D>;
  T qr[C::ROW_ELEMS];    // Q rows   [32][D]
  T dr[C::ROW_ELEMS];    // dO rows  [32][D]
  T qt[C::COL_ELEMS];    // Q^T      [D][32]
  T dt[C::COL_ELEMS];    // dO^T     [D][32]
  float c[32], dot[32];
};

// Read-only inputs of the query side.
template <typename T> struct QSide {
  const T* q;
  const T* dout;
  const T* qt;     // [B][Hkv][NHC][T][D][16]
  const T* dt;
  const float* lse;
  const float* dot;
  const float* rowscale;
  int Hq, Hkv, G, NHC, T_;
};

// Loads of one 2-query row tile: the four operand tiles go straight to LDS;
// the row statistics are loaded into registers by threads 0..31 and written
// (combined) after the tile in flight has been consumed.
template <typename T, int D, int NTH> struct RowTileLoader {
  using C = Tile32<T, D>;
  float lse_, rs_, dot_;
  bool ok_;

  __device__ __forceinline__ void issue(KvStage<T, D>& s, const QSide<T>& x, int b, int hkv, int hc, int tA, int tB,
                                        int tid) {
    const int tq[2] = {tA, tB >= 0 ? tB : tA};      // a missing second query re-reads the first
    const int grem = x.G - hc * 16;                   // heads of this chunk
    const int64_t hbase = (int64_t)b * x.Hq + hkv * x.G + hc * 16;
    const int64_t cbase = (((int64_t)b * x.Hkv + hkv) * x.NHC + hc) * x.T_;
    auto rows = [&](const T* src) {
      return [&, src](int P) {
        int r, cc;
        row_chunk<T, D>(P, r, cc);
        const int hd = (r & 15) < grem ? (r & 15) : grem - 1;
        return (const void*)(src + ((hbase + hd) * x.T_ + tq[r >> 4]) * D + cc * C::EPC);
      };
    };
    auto cols = [&](const T* src) {
      return [&, src](int P) {
        int d, cc;
        col_chunk<T, D>(P, d, cc);
        const int r0 = cc * C::EPC;
        return (const void*)(src + ((cbase + tq[r0 >> 4]) * D + d) * 16 + (r0 & 15));
      };
    };
    dma_tile<NTH, C::ROW_CHUNKS>(s.qr, rows(x.q), tid);
    dma_tile<NTH, C::ROW_CHUNKS>(s.dr, rows(x.dout), tid);
    dma_tile<NTH, C::COL_CHUNKS>(s.qt, cols(x.qt), tid);
    dma_tile<NTH, C::COL_CHUNKS>(s.dt, cols(x.dt), tid);
    if (tid < 32) {
      const int t = tid < 16 ? tA : tB;
      const int hd = tid & 15;
      ok_ = t >= 0 && hd < grem;
      const int64_t ri = (hbase + (hd < grem ? hd : grem - 1)) * x.T_ + (t >= 0 ? t : tA);
      lse_ = x.lse[ri];
      rs_ = x.rowscale != nullptr ? x.rowscale[ri] : 1.0f;
      dot_ = x.dot[ri];
    }
  }

  __device__ __forceinline__ void finish(KvStage<T, D>& s, int tid) const {
    if (tid < 32) {
      s.c[tid] = ok_ ? lse_ * kLog2e - __log2f(rs_) : __builtin_inff();
      s.dot[tid] = dot_;
    }
  }
};

// Per-wave key state: 32 keys, their K / V fragments and dK^T / dV^T.
template <typename T, int D> struct KeyAcc {
  using C = Tile32<T, D>;
  Frag<T> kf[C::KS], vf[C::KS];
  f32x16 dk[C::DT], dv[C::DT];

  // keys past the end read key `key_safe`: finite data whose columns are never stored
  __device__ __forceinline__ void init(const T* kb, const T* vb, int key_safe, int h) {
#pragma unroll
    for (int s = 0; s < C::KS; ++s) {
      kf[s].load(kb + (int64_t)key_safe * D + 16 * s + 8 * h);
      vf[s].load(vb + (int64_t)key_safe * D + 16 * s + 8 * h);
    }
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
      dk[dt] = zero16();
      dv[dt] = zero16();
    }
  }

  // One 2-query tile; with `mask`, visA / visB say whether this lane's key is
  // visible to query A / B.
  __device__ __forceinline__ void step(const KvStage<T, D>& s, bool mask, bool visA, bool visB, float sl2, int n,
                                       int h, float* ds_out = nullptr) {
    // every operand fragment of the tile is read up front so the LDS reads
    // overlap each other and the MFMAs
    Frag<T> qa[C::KS], da[C::KS];
#pragma unroll
    for (int k = 0; k < C::KS; ++k) {
      lds_row_frag<T, D>(qa[k], s.qr, n, h, k);
      lds_row_frag<T, D>(da[k], s.dr, n, h, k);
    }
    f32x16 sacc = zero16(), pacc = zero16();
#pragma unroll
    for (int k = 0; k < C::KS; ++k) {
      mma32(sacc, qa[k], kf[k]);
      mma32(pacc, da[k], vf[k]);
    }
    Frag<T> ta[C::DT][2], tb[C::DT][2];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        lds_col_frag<T, D>(ta[dt][k], s.dt, dt, n, h, k);
        lds_col_frag<T, D>(tb[dt][k], s.qt, dt, n, h, k);
      }
    float P[16], dS[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int e = acc_elem(h, r);
      float p = fast_exp2(sacc[r] * sl2 - s.c[e]);
      if (mask) p = (r < 8 ? visA : visB) ? p : 0.0f;
      P[r] = p;
      dS[r] = p * (pacc[r] - s.dot[e]);
    }
    if (ds_out != nullptr) {
#pragma unroll
      for (int r = 0; r < 16; ++r) ds_out[r] = dS[r];
    }
    Frag<T> pf[2], sf[2];
    pf[0].set(P);
    pf[1].set(P + 8);
    sf[0].set(dS);
    sf[1].set(dS + 8);
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        mma32(dv[dt], ta[dt][k], pf[k]);
        mma32(dk[dt], tb[dt][k], sf[k]);
      }
    }
  }

  __device__ __forceinline__ void write(float* dkrow, float* dvrow, float scale, bool atomic, int h) const {
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * h;
        if (!(D % 32 == 0 || d < D)) continue;
        if (atomic) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            atomicAdd(dkrow + d + i, dk[dt][4 * g4 + i] * scale);
            atomicAdd(dvrow + d + i, dv[dt][4 * g4 + i]);
          }
        } else {
          *reinterpret_cast<f32x4*>(dkrow + d) = (f32x4){dk[dt][4 * g4], dk[dt][4 * g4 + 1], dk[dt][4 * g4 + 2],
                                                         dk[dt][4 * g4 + 3]} * scale;
          *reinterpret_cast<f32x4*>(dvrow + d) =
              (f32x4){dv[dt][4 * g4], dv[dt][4 * g4 + 1], dv[dt][4 * g4 + 2], dv[dt][4 * g4 + 3]};
        }
      }
    }
  }
};

// Walk `ntile` 2-query tiles (queries and their block_idx slots from
// qsrc(i, tA, tB, sA, sB); tB = -1: none) over every head chunk,
// double-buffered.  vis(tA, tB, mask, visA, visB) fills the mask flags of a
// tile for this wave.  post(tA, tB, sA, sB, hc, dS) runs on every thread of
// the workgroup after each tile's step with this lane's 16 dS values (it may
// synchronise the workgroup); WANT_DS = false skips it.
template <bool WANT_DS, typename T, int D, int NTH, typename QSrc, typename Vis, typename Post>
__device__ __forceinline__ void kv_walk(KeyAcc<T, D>& acc, KvStage<T, D> (&stg)[2], const QSide<T>& x, int b,
                                        int hkv, int ntile, QSrc qsrc, Vis vis, Post post, float sl2, int tid, int n,
                                        int h) {
  RowTileLoader<T, D, NTH> ld;
  const int total = ntile * x.NHC;
  if (total == 0) return;
  {
    int tA, tB, sA, sB;
    qsrc(0, tA, tB, sA, sB);
    ld.issue(stg[0], x, b, hkv, 0, tA, tB, tid);
    ld.finish(stg[0], tid);
  }
  lds_dma_wait();
  __syncthreads();
  int ti = 0, hc = 0;   // tile and head chunk of iteration `it`
  for (int it = 0; it < total; ++it) {
    int tA, tB, sA, sB;
    qsrc(ti, tA, tB, sA, sB);
    int ti1 = ti + 1, hc1 = hc;
    if (ti1 == ntile) {
      ti1 = 0;
      ++hc1;
    }
    if (it + 1 < total) {
      int uA, uB, vA, vB;
      qsrc(ti1, uA, uB, vA, vB);
      ld.issue(stg[(it + 1) & 1], x, b, hkv, hc1, uA, uB, tid);
    }
    bool mask, visA, visB;
    vis(tA, tB, mask, visA, visB);
    float ds[16];
    acc.step(stg[it & 1], mask, visA, visB, sl2, n, h, WANT_DS ? ds : nullptr);
    if (WANT_DS) post(tA, tB, sA, sB, hc, ds);
    if (it + 1 < total) ld.finish(stg[(it + 1) & 1], tid);
    lds_dma_wait();
    __syncthreads();
    ti = ti1;
    hc = hc1;
  }
}

template <typename T>
__device__ __forceinline__ QSide<T> qside(const T* q, const T* dout, const T* qt, const T* dt, const float* lse,
                                          const float* dot, const float* rowscale, int Hq, int Hkv, int T_) {
  QSide<T> x;
  x.q = q;
  x.dout = dout;
  x.qt = qt;
  x.dt = dt;
  x.lse = lse;
  x.dot = dot;
  x.rowscale = rowscale;
  x.Hq = Hq;
  x.Hkv = Hkv;
  x.G = Hq / Hkv;
  x.NHC = (x.G + 15) / 16;
  x.T_ = T_;
  return x;
}

// ---------------------------------------------------------------------------
// range dK/dV: grid (ceil(Lk / (32 NW)), n_chunks, B*Hkv)
// ---------------------------------------------------------------------------
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) void k_range_dkdv32(int mode, const T* __restrict__ q,
                                                          const T* __restrict__ dout, const T* __restrict__ qt,
                                                          const T* __restrict__ dt, const float* __restrict__ lse,
                                                          const float* __restrict__ dot,
                                                          const float* __restrict__ rowscale,
                                                          const T* __restrict__ k, const T* __restrict__ v,
                                                          float* __restrict__ dk, float* __restrict__ dv, int Hq,
                                                          int Hkv, int T_, int Lk, int chunk, int window, int cl,
                                                          int cd, float sl2, float scale) {
  constexpr int NTH = 64 * NW;
  __shared__ __align__(16) KvStage<T, D> stg[2];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const int bh = blockIdx.z;
  const int b = bh / Hkv, hkv = bh % Hkv;
  const int k0 = blockIdx.x * 32 * NW;
  const int kw = k0 + 32 * w;
  const int key = kw + n;
  const bool key_ok = key < Lk;
  const QSide<T> x = qside(q, dout, qt, dt, lse, dot, rowscale, Hq, Hkv, T_);
  // query range of the workgroup
  int tlo, thi;
  const int klast = k0 + 32 * NW - 1 < Lk - 1 ? k0 + 32 * NW - 1 : Lk - 1;
  if (mode == NSA_MODE_WINDOW) {
    tlo = k0;
    thi = klast + window - 1;
  } else {
    tlo = k0 * cd + cl - 1;
    thi = T_ - 1;
    const int c0 = blockIdx.y * chunk, c1 = c0 + chunk - 1;
    tlo = tlo > c0 ? tlo : c0;
    thi = thi < c1 ? thi : c1;
  }
  thi = thi < T_ - 1 ? thi : T_ - 1;
  if (tlo > thi) return;   // uniform over the workgroup
  KeyAcc<T, D> acc;
  const int64_t kvoff = (int64_t)bh * Lk * D;
  acc.init(k + kvoff, v + kvoff, key_ok ? key : Lk - 1, h);
  const int ntile = (thi - tlo) / 2 + 1;
  const int wlast = kw + 31;   // last key of the wave (may pass Lk: those columns are never stored)
  auto qsrc = [&](int i, int& tA, int& tB, int& sA, int& sB) {
    tA = tlo + 2 * i;
    tB = tA + 1 <= thi ? tA + 1 : -1;
    sA = sB = 0;
  };
  auto vis = [&](int tA, int tB, bool& mask, bool& visA, bool& visB) {
    const int tb = tB >= 0 ? tB : tA;
    if (mode == NSA_MODE_WINDOW) {
      mask = !(tA >= wlast && tb - window < kw);
      visA = key <= tA && key > tA - window;
      visB = key <= tb && key > tb - window;
    } else {
      mask = !(wlast * cd + cl - 1 <= tA);
      visA = key * cd + cl - 1 <= tA;
      visB = key * cd + cl - 1 <= tb;
    }
  };
  auto none = [](int, int, int, int, int, const float*) {};
  kv_walk<false, T, D, NTH>(acc, stg, x, b, hkv, ntile, qsrc, vis, none, sl2, tid, n, h);
  if (key_ok) acc.write(dk + kvoff + (int64_t)key * D, dv + kvoff + (int64_t)key * D, scale,
                        mode == NSA_MODE_COMPRESS, h);
}

__global__ __launch_bounds__(256) void k_fill_zero(float* __restrict__ x, int64_t n) {
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) x[e] = 0.0f;
}

// Zero-fill with a kernel (safe inside captured graphs, unlike a memset node).
static inline int zero_f32(float* x, int64_t n, hipStream_t s) {
  if (n <= 0) return NSA_OK;
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  k_fill_zero<<<(unsigned)g, 256, 0, s>>>(x, n);
  return hipGetLastError() == hipSuccess ? NSA_OK : NSA_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// selection dK/dV over CSR work items (nsa_items.h)
// ---------------------------------------------------------------------------
// Persistent grid over the work items; two waves own 64 keys of the item's
// block at a time (blocks longer than 64 keys take several passes).  With
// dq_part, the tile's dS (both waves, 32 rows x 64 keys) is staged in LDS and
// dQ^T = K^T dS^T is formed for the pass's 64 keys -- each wave covering half
// of D -- and written, scaled, to the (query, slot, pass) partial that
// k_sel_dq_reduce sums.
template <typename T, int D>
__global__ __launch_bounds__(128) void k_sel_dkdv32(const T* __restrict__ q, const T* __restrict__ dout,
                                                    const T* __restrict__ qt, const T* __restrict__ dt,
                                                    const float* __restrict__ lse, const float* __restrict__ dot,
                                                    const float* __restrict__ rowscale, const T* __restrict__ k,
                                                    const T* __restrict__ v, const T* __restrict__ kt,
                                                    const int32_t* __restrict__ q_of_block,
                                                    const int4* __restrict__ items,
                                                    const int32_t* __restrict__ n_items, float* __restrict__ dk,
                                                    float* __restrict__ dv, T* __restrict__ dq_part, int Hq, int Hkv,
                                                    int T_, int S, int packed, int n_blk, int L, int Lp, float sl2,
                                                    float scale) {
  constexpr int NW = 2, NTH = 64 * NW;
  using C = Tile32<T, D>;
  constexpr int DT = C::DT, DTW = (DT + 1) / 2;          // dQ^T d-tiles per wave
  constexpr int DSP = 64 + 16 / (int)sizeof(T);          // padded pitch of the dS tile
  __shared__ __align__(16) KvStage<T, D> stg[2];
  __shared__ __align__(16) T sdS[32 * DSP];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const QSide<T> x = qside(q, dout, qt, dt, lse, dot, rowscale, Hq, Hkv, T_);
  const int G = x.G;
  const int ni = *n_items;
  const int npass = sel_passes(L);
  const int NS = S * npass;
  for (int it = blockIdx.x; it < ni * npass; it += gridDim.x) {
    const int4 item = items[it / npass];
    const int pass = it % npass;
    const int bh = item.x / n_blk, j = item.x % n_blk;
    const int b = bh / Hkv, hkv = bh % Hkv;
    const int blk_end = j * L + L < T_ ? j * L + L : T_;
    const int kpass = j * L + kSelPass * pass;
    const int kw = kpass + 32 * w;
    const int key = kw + n;
    const bool key_ok = key < blk_end;
    const int wlast = kw + 31;
    const int64_t kvoff = (int64_t)bh * T_ * D;
    KeyAcc<T, D> acc;
    acc.init(k + kvoff, v + kvoff, key_ok ? key : j * L, h);
    // K^T fragments of the pass's 64 keys for this wave's dQ^T d-tiles
    Frag<T> ktf[DTW][4];
    if (dq_part != nullptr) {
      const T* ktb = kt + (int64_t)bh * D * Lp;
#pragma unroll
      for (int i = 0; i < DTW; ++i)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int d = 32 * (w * DTW + i) + n;
          int c0 = kpass + 16 * kk + 8 * h;
          c0 = c0 < Lp - 8 ? c0 : Lp - 8;
          if (w * DTW + i < DT && (D % 32 == 0 || d < D))
            ktf[i][kk].load(ktb + (int64_t)d * Lp + c0);
          else
            ktf[i][kk].zero();
        }
    }
    const int beg = item.y, cnt = item.z - item.y;
    const int ntile = (cnt + 1) / 2;
    auto decode = [&](int i, int& t, int& s) {
      if (i < cnt) {
        const int val = q_of_block[beg + i];
        t = packed ? val / S : val;
        s = packed ? val % S : 0;
      } else {
        t = -1;
        s = 0;
      }
    };
    auto qsrc = [&](int i, int& tA, int& tB, int& sA, int& sB) {
      decode(2 * i, tA, sA);
      decode(2 * i + 1, tB, sB);
    };
    auto vis = [&](int tA, int tB, bool& mask, bool& visA, bool& visB) {
      const int tb = tB >= 0 ? tB : tA;
      mask = !(wlast <= tA && wlast < blk_end);
      visA = key_ok && key <= tA;
      visB = key_ok && key <= tb;
    };
    auto post = [&](int tA, int tB, int sA, int sB, int hc, const float* ds) {
      // dS (rows x this wave's 32 keys) -> LDS [row][64 keys]
#pragma unroll
      for (int r = 0; r < 16; ++r) sdS[acc_elem(h, r) * DSP + 32 * w + n] = from_f32<T>(ds[r]);
      __syncthreads();
      f32x16 dq[DTW];
#pragma unroll
      for (int i = 0; i < DTW; ++i) dq[i] = zero16();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        Frag<T> bf;
        const T* src = sdS + n * DSP + 16 * kk + 8 * h;
        if (sizeof(T) == 2)
          bf.load(src);
        else
          bf.load2(src, src + 4);
#pragma unroll
        for (int i = 0; i < DTW; ++i) mma32(dq[i], ktf[i][kk], bf);
      }
      const int t = n < 16 ? tA : tB;
      const int g = hc * 16 + (n & 15);
      if (t >= 0 && g < G) {
        const int slot = (n < 16 ? sA : sB) * npass + pass;
        T* drow = dq_part + ((((int64_t)bh * T_ + t) * NS + slot) * G + g) * D;
#pragma unroll
        for (int i = 0; i < DTW; ++i) {
          if (w * DTW + i >= DT) continue;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int d = 32 * (w * DTW + i) + 8 * g4 + 4 * h;
            if (D % 32 == 0 || d < D)
              store4(drow + d, dq[i][4 * g4] * scale, dq[i][4 * g4 + 1] * scale, dq[i][4 * g4 + 2] * scale,
                     dq[i][4 * g4 + 3] * scale);
          }
        }
      }
    };
    if (dq_part != nullptr)
      kv_walk<true, T, D, NTH>(acc, stg, x, b, hkv, ntile, qsrc, vis, post, sl2, tid, n, h);
    else
      kv_walk<false, T, D, NTH>(acc, stg, x, b, hkv, ntile, qsrc, vis, post, sl2, tid, n, h);
    if (key_ok) acc.write(dk + kvoff + (int64_t)key * D, dv + kvoff + (int64_t)key * D, scale, true, h);
    __syncthreads();   // the next item's first tile reuses stage 0
  }
}

}  // namespace nsa

using namespace nsa;

#define NSA_DISPATCH_D(D_, ...)                                 \
  switch (D_) {                                                 \
    case 16: { constexpr int DD = 16; __VA_ARGS__; break; }    \
    case 32: { constexpr int DD = 32; __VA_ARGS__; break; }    \
    case 64: { constexpr int DD = 64; __VA_ARGS__; break; }    \
    case 128: { constexpr int DD = 128; __VA_ARGS__; break; }  \
    default: return NSA_ERR_SHAPE;                              \
  }

static constexpr int kCmpChunk = 1024;   // queries per compression dK/dV work item


extern "C" {

int nsa_range_dkdv(int mode, const void* q, const void* k, const void* v, const void* dout, const void* qt,
                   const void* dout_t, const float* lse, const float* dot, const float* rowscale, float* dk,
                   float* dv, int B, int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block,
                   int cmp_stride, int dtype, void* stream) {
  NSA_CHECK(mode == NSA_MODE_WINDOW || mode == NSA_MODE_COMPRESS, NSA_ERR_ARG);
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && Lk >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(mode == NSA_MODE_COMPRESS || (window >= 1 && Lk == T), NSA_ERR_SHAPE);
  NSA_CHECK(mode == NSA_MODE_WINDOW || (cmp_block >= 1 && cmp_stride >= 1), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  hipStream_t s = (hipStream_t)stream;
  const int64_t nel = (int64_t)B * Hkv * Lk * D;
  if (mode == NSA_MODE_COMPRESS || T == 0) {
    if (zero_f32(dk, nel, s) != NSA_OK || zero_f32(dv, nel, s) != NSA_OK) return NSA_ERR_LAUNCH;
  }
  if (T == 0 || Lk == 0) return NSA_OK;
  const int nch = mode == NSA_MODE_COMPRESS ? (T + kCmpChunk - 1) / kCmpChunk : 1;
  NSA_CHECK((int64_t)B * Hkv < 65536, NSA_ERR_SHAPE);
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  // window: 2 waves (64 keys) per workgroup keep the query range tight;
  // compression: 4 waves share each streamed query tile
#define NSA_RANGE_DKDV_LAUNCH(NW_)                                                                               \
  {                                                                                                            \
    dim3 grid((Lk + 32 * NW_ - 1) / (32 * NW_), nch, B * Hkv);                                                  \
    NSA_DISPATCH_D(D, {                                                                                        \
      if (dtype == NSA_BF16)                                                                                   \
        k_range_dkdv32<bf16, DD, NW_><<<grid, 64 * NW_, 0, s>>>(                                               \
            mode, (const bf16*)q, (const bf16*)dout, (const bf16*)qt, (const bf16*)dout_t, lse, dot, rowscale, \
            (const bf16*)k, (const bf16*)v, dk, dv, Hq, Hkv, T, Lk, kCmpChunk, window, cmp_block, cmp_stride,  \
            sl2, scale);                                                                                       \
      else                                                                                                     \
        k_range_dkdv32<float, DD, NW_><<<grid, 64 * NW_, 0, s>>>(                                              \
            mode, (const float*)q, (const float*)dout, (const float*)qt, (const float*)dout_t, lse, dot,        \
            rowscale, (const float*)k, (const float*)v, dk, dv, Hq, Hkv, T, Lk, kCmpChunk, window, cmp_block,  \
            cmp_stride, sl2, scale);                                                                           \
    });                                                                                                        \
  }
  if (mode == NSA_MODE_WINDOW)
    NSA_RANGE_DKDV_LAUNCH(2)
  else
    NSA_RANGE_DKDV_LAUNCH(4)
#undef NSA_RANGE_DKDV_LAUNCH
  return nsa_launch_status();
}

size_t nsa_sel_dkdv_workspace(int B, int Hkv, int T, int S, int block_size, int chunk) {
  if (B <= 0 || Hkv <= 0 || T < 0 || S < 0 || block_size <= 0 || chunk <= 0) return 0;
  return sel_items_cap(B, Hkv, T, S, block_size, chunk) * sizeof(int4) + 256;
}

int nsa_sel_dkdv(const void* q, const void* k, const void* v, const void* kt, const void* dout, const void* qt,
                 const void* dout_t, const float* lse, const float* dot, const float* rowscale,
                 const int32_t* q_of_block, int packed, const int32_t* block_offsets, const int32_t* pair_count,
                 float* dk, float* dv, void* dq_part, void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv,
                 int T, int D, int S, int block_size, int chunk, int dtype, void* stream) {
  (void)pair_count;
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && S >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(block_size >= 16 && block_size % 16 == 0 && chunk >= 2, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(workspace_bytes >= nsa_sel_dkdv_workspace(B, Hkv, T, S, block_size, chunk), NSA_ERR_WORKSPACE);
  NSA_CHECK(dq_part == nullptr || (packed && kt != nullptr), NSA_ERR_ARG);
  NSA_CHECK(!packed || (int64_t)T * S < (1ll << 31), NSA_ERR_SHAPE);
  hipStream_t s = (hipStream_t)stream;
  const int64_t nel = (int64_t)B * Hkv * T * D;
  if (zero_f32(dk, nel, s) != NSA_OK || zero_f32(dv, nel, s) != NSA_OK) return NSA_ERR_LAUNCH;
  const int n_blk = sel_csr_blocks(T, block_size);
  if (T == 0 || S == 0 || n_blk == 0) return NSA_OK;
  const size_t cap = sel_items_cap(B, Hkv, T, S, block_size, chunk);
  int4* items = (int4*)workspace;
  int32_t* n_items = (int32_t*)((char*)workspace + cap * sizeof(int4));
  k_sel_items<<<1, 1024, 0, s>>>(block_offsets, B * Hkv * n_blk, n_blk, chunk, items, n_items);
  if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
  const size_t grid_cap = cap * sel_passes(block_size) < 4096 ? cap * sel_passes(block_size) : 4096;
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  const int Lp = padded_len(T);
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16)
      k_sel_dkdv32<bf16, DD><<<(unsigned)grid_cap, 128, 0, s>>>(
          (const bf16*)q, (const bf16*)dout, (const bf16*)qt, (const bf16*)dout_t, lse, dot, rowscale,
          (const bf16*)k, (const bf16*)v, (const bf16*)kt, q_of_block, items, n_items, dk, dv, (bf16*)dq_part, Hq,
          Hkv, T, S, packed, n_blk, block_size, Lp, sl2, scale);
    else
      k_sel_dkdv32<float, DD><<<(unsigned)grid_cap, 128, 0, s>>>(
          (const float*)q, (const float*)dout, (const float*)qt, (const float*)dout_t, lse, dot, rowscale,
          (const float*)k, (const float*)v, (const float*)kt, q_of_block, items, n_items, dk, dv, (float*)dq_part,
          Hq, Hkv, T, S, packed, n_blk, block_size, Lp, sl2, scale);
  });
  return nsa_launch_status();
}

}  // extern "C"
