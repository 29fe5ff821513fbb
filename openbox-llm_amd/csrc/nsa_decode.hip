// Decode: one new query per sequence against its KV caches -- the three NSA
// branches, block importance and top-n for a single query position t = len-1
// (no counterpart in the reference, which runs whole sequences; the
// semantics are those of NSAAttention at row t, nsa_model.py:196-304, with
// the candidate blocks 0 .. t / l' that a sequence reaching past block t / l'
// offers: a decode step equals row t of any prefill whose length covers the
// end of t's selection block).
//
// Five launches on the caller's stream, no host synchronisation (four when
// the pooled sequence fits two token-sum chunks, <= 2048 tokens: k_dec_topn
// then forms the token sums itself, with k_dec_toksum's arithmetic):
//  1. k_dec_part (compression + window): split-K over the pooled tokens and
//     the window keys.  One wave per split (up to 8 tiles of 32 keys; fewer
//     when the batch is small, so the splits still spread over the CUs).
//     K and V tiles go global -> LDS by direct loads (two stages per wave),
//     S^T = K Q^T puts the group's heads on the MFMA columns, P V^T reads the
//     V row tile through ds_read_b64_tr_b16.  Each split writes an
//     unnormalised partial (running max in log2 units, sum, output);
//     compression splits also write their raw scores, so the importance
//     never re-reads the pooled keys.
//  2. k_dec_toksum: per 1024 pooled tokens, each head's log-sum-exp from the
//     compression splits, then p_cmp summed over the group's heads per token
//     (heads 0-7 then 8-15 of each 16-head chunk, as the prefill importance
//     kernel sums them).
//  3. k_dec_topn: one workgroup per (b, hkv) folds the token sums into the
//     candidate blocks (overlap / cmp_stride), masks and forces them, and
//     selects the top S with ties to the lower block by radix selection on
//     64-bit (score, ~block) keys.
//  4. k_dec_part (selection): split-K over the picked blocks.
//  5. k_dec_merge: per query head, one wave per branch combines its partials;
//     the gated sum adds the branches in gate order.
#include "nsa_launch.h"
#include "nsa_tile32.h"

namespace nsa {

constexpr int kDecMaxTiles = 8;     // most 32-key tiles per split (compression; 4 window / selection)
constexpr int kDecMaxCand = 4096;   // candidate blocks per query (4 keys per top-n thread)
constexpr float kDecNegInf = -__builtin_inff();
constexpr float kDecRescale = 8.0f;   // log2 growth of a running maximum that forces a rescale

struct DecGeom {
  int B, Hq, Hkv, G, NHC;   // NHC: head chunks of 32 (MFMA columns)
  int Tcap, Ncap, NcapP;    // cache capacities; NcapP: score row pitch (multiple of 32)
  int cl, cd, ls, tpb;      // compression span / stride, selection block, tiles per block
  int n_sel, window, force_init, n_local;
  int ct, wt, st;           // tiles per split: compression, window, selection
  int ncs, nws, nss;        // splits per branch at the longest length
};

// Per-sequence quantities of query position t = len - 1.
struct DecLen {
  int len, t;
  int nvis;          // pooled tokens visible: i * cd + cl - 1 <= t
  int wlo, wkt0;     // window keys [wlo, t]; first tile starts at wkt0
  int nwt;           // window tiles
  int ncand, S;      // candidate blocks 0 .. t / ls; picks
};

__host__ __device__ inline DecLen dec_len(int len, const DecGeom& g) {
  DecLen L;
  len = len < 0 ? 0 : (len > g.Tcap ? g.Tcap : len);
  L.len = len;
  L.t = len - 1;
  const int t = L.t;
  if (t < 0) {
    L.nvis = L.wlo = L.wkt0 = L.nwt = L.ncand = L.S = 0;
    return L;
  }
  L.nvis = t >= g.cl - 1 ? (t - g.cl + 1) / g.cd + 1 : 0;
  L.wlo = t - g.window + 1 > 0 ? t - g.window + 1 : 0;
  L.wkt0 = L.wlo & ~31;
  L.nwt = (t - L.wkt0) / 32 + 1;
  L.ncand = t / g.ls + 1;
  L.S = g.n_sel < L.ncand ? g.n_sel : L.ncand;
  return L;
}

// splits each branch uses at this length
__host__ __device__ inline int dec_cmp_splits(const DecLen& L, const DecGeom& g) {
  return ((L.nvis + 31) / 32 + g.ct - 1) / g.ct;
}
__host__ __device__ inline int dec_win_splits(const DecLen& L, const DecGeom& g) { return (L.nwt + g.wt - 1) / g.wt; }
__host__ __device__ inline int dec_sel_splits(const DecLen& L, const DecGeom& g) {
  return (L.S * g.tpb + g.st - 1) / g.st;
}

template <typename T>
struct DecArgs {
  const T* q;         // [B][Hq][D]
  const T* kcmp;      // [B][Hkv][Ncap][D]
  const T* vcmp;
  const T* ks;        // [B][Hkv][Tcap][D]
  const T* vs;
  const T* kw;
  const T* vw;
  const T* gate;      // [B][Hq][3]
  const int32_t* lens;
  T* out;             // [B][Hq][D]
  int32_t* idx;       // [B][Hkv][n_sel]
  float* scores;      // nullable [B][Hkv][ncand_cap]
  float* o_branch;    // nullable [3][B][Hq][D]
  float* lse_branch;  // nullable [3][B][Hq]
  float* p1_ml;       // [NG][ncs + nws][32][2]  (NG = B * Hkv * NHC)
  float* p1_o;        // [NG][ncs + nws][32][D]
  float* p3_ml;       // [NG][nss][32][2]
  float* p3_o;        // [NG][nss][32][D]
  float* s_cmp;       // [B * Hkv][G][NcapP] raw compression scores
  float* tok;         // [B * Hkv][NcapP] p_cmp summed over the group's heads
  int ncand_cap;
  float sl2;          // D^-1/2 * log2(e)
  DecGeom g;
};

// One 32-key tile: S^T = K Q^T (keys on M, heads on N), online softmax per
// head column, O^T += V^T P.  Keys outside [lo, hi] are masked.  srow
// (nullable): this lane's head row of raw scores, written for the whole tile.
template <typename T, int D, int DT = Tile32<T, D>::DT, int KS = Tile32<T, D>::KS>
__device__ __forceinline__ void dec_tile(f32x16 (&acc)[DT], float& m_, float& l_, const Frag<T> (&qf)[KS],
                                         const T* tK, const T* tV, int kb, int lo, int hi, float sl2, int lane,
                                         float* srow) {
  using C = Tile32<T, D>;
  const int h = lane >> 5, n = lane & 31;
  Frag<T> ka[C::KS];
#pragma unroll
  for (int s = 0; s < C::KS; ++s) lds_row_frag<T, D>(ka[s], tK, n, h, s);
  f32x16 st = zero16();
#pragma unroll
  for (int s = 0; s < C::KS; ++s) mma32(st, ka[s], qf[s]);
  Frag<T> va[C::DT][2];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) lds_tr_frag<T, D>(va[dt][s], tV, dt, lane, s);
  if (srow != nullptr) {
    // registers 8u .. 8u+7 hold keys kb + 16u + 8h .. +7
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float* p = srow + kb + 16 * u + 8 * h;
      *reinterpret_cast<f32x4*>(p) = (f32x4){st[8 * u], st[8 * u + 1], st[8 * u + 2], st[8 * u + 3]};
      *reinterpret_cast<f32x4*>(p + 4) = (f32x4){st[8 * u + 4], st[8 * u + 5], st[8 * u + 6], st[8 * u + 7]};
    }
  }
  if (kb < lo || kb + 31 > hi) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + acc_elem(h, r);
      st[r] = (key >= lo && key <= hi) ? st[r] : kDecNegInf;
    }
  }
  float v = st[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) v = fmaxf(v, st[r]);
  const float mx = fmaxf(v, __shfl_xor(v, 32, kWave)) * sl2;
  if (mx > m_ + kDecRescale) {
    const float alpha = fast_exp2(m_ - mx);
    l_ *= alpha;
    m_ = mx;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
  }
  float p[16];
  float ps = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    p[r] = fast_exp2(st[r] * sl2 - m_);
    ps += p[r];
  }
  l_ += ps;
  Frag<T> pf[2];
  pf[0].set(p);
  pf[1].set(p + 8);
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) mma32(acc[dt], va[dt][s], pf[s]);
}

// Branch numbering follows the gate: 0 compression, 1 selection, 2 window.
template <typename T, int D, int NST>
__global__ __launch_bounds__(64) void k_dec_part(const DecArgs<T> a, int sel_phase) {
  using C = Tile32<T, D>;
  __shared__ __align__(16) T sK[NST][C::ROW_ELEMS];
  __shared__ __align__(16) T sV[NST][C::ROW_ELEMS];
  const DecGeom& g = a.g;
  const int lane = threadIdx.x, h = lane >> 5, n = lane & 31;
  const int nsp = sel_phase ? g.nss : g.ncs + g.nws;
  const int split = (int)(blockIdx.x % (unsigned)nsp);
  const int grp = (int)(blockIdx.x / (unsigned)nsp);   // (b * Hkv + hkv) * NHC + hc
  const int hc = grp % g.NHC, bh = grp / g.NHC;
  const int b = bh / g.Hkv, hkv = bh % g.Hkv;
  const DecLen L = dec_len(a.lens[b], g);
  if (L.t < 0) return;
  int branch, t0, nt;   // tiles t0 .. t0 + nt - 1 of the branch's tile list
  if (sel_phase) {
    branch = 1;
    t0 = split * g.st;
    nt = L.S * g.tpb - t0;
    nt = nt < g.st ? nt : g.st;
  } else if (split < g.ncs) {
    branch = 0;
    t0 = split * g.ct;
    nt = (L.nvis + 31) / 32 - t0;
    nt = nt < g.ct ? nt : g.ct;
  } else {
    branch = 2;
    t0 = (split - g.ncs) * g.wt;
    nt = L.nwt - t0;
    nt = nt < g.wt ? nt : g.wt;
  }
  if (nt <= 0) return;

  const int64_t kvoff = branch == 0 ? (int64_t)bh * g.Ncap * D : (int64_t)bh * g.Tcap * D;
  const T* kbase = (branch == 0 ? a.kcmp : branch == 1 ? a.ks : a.kw) + kvoff;
  const T* vbase = (branch == 0 ? a.vcmp : branch == 1 ? a.vs : a.vw) + kvoff;
  const int nrows = branch == 0 ? L.nvis : L.len;   // rows past the last valid one repeat it
  const int32_t* sidx = a.idx + (int64_t)bh * g.n_sel;
  // tile i of this split: first row r0 and visible keys [lo, hi]
  auto tile_of = [&](int i, int& r0, int& lo, int& hi) {
    const int u = t0 + i;
    if (branch == 0) {
      r0 = 32 * u;
      lo = 0;
      hi = L.nvis - 1;
    } else if (branch == 2) {
      r0 = L.wkt0 + 32 * u;
      lo = L.wlo;
      hi = L.t;
    } else {
      const int j = __builtin_amdgcn_readfirstlane(sidx[u / g.tpb]);
      const int base = j * g.ls;
      r0 = base + 32 * (u % g.tpb);
      lo = base;
      hi = base + g.ls - 1 < L.t ? base + g.ls - 1 : L.t;
      if (j < 0 || r0 > L.t) {   // no visible key: any valid row, all masked
        r0 = 0;
        lo = 1;
        hi = 0;
      }
    }
  };

  const int Gc = g.G - 32 * hc < 32 ? g.G - 32 * hc : 32;   // heads of this chunk
  const int hd = n < Gc ? n : 0;
  const T* qrow = a.q + ((int64_t)b * g.Hq + hkv * g.G + 32 * hc + hd) * D;
  RowTileDma<T, D, 64, false> dma;   // K and V rows share the per-lane offsets
  dma.init(lane);
  constexpr int LT = 2 * decltype(dma)::NL;   // vector-memory loads per tile
  static_assert((NST - 1) * LT + 4 < 64, "in-flight operations exceed the vmcnt range");
  auto request = [&](int i) {
    int r0, lo, hi;
    tile_of(i, r0, lo, hi);
    dma.request(sK[i % NST], kbase, r0, nrows, lane);
    dma.request(sV[i % NST], vbase, r0, nrows, lane);
  };
  // the first tiles go out before the Q loads, so one memory latency covers
  // both (the wait the compiler puts before the first use of Q also covers
  // these tiles, which it does not see)
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < nt) request(p);
  Frag<T> qf[C::KS];
#pragma unroll
  for (int s = 0; s < C::KS; ++s) qf[s].load(qrow + 16 * s + 8 * h);
#pragma unroll
  for (int s = 0; s < C::KS; ++s) settle(qf[s]);
  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = zero16();
  float m_ = kMaskScore, l_ = 0.0f;
  float* srow = branch == 0 && n < Gc ? a.s_cmp + ((int64_t)bh * g.G + 32 * hc + n) * g.NcapP : nullptr;
  // tile it: wait for it (the NST-2 younger tiles stay in flight), refill the
  // stage of tile it-1 (read by this wave only, its reads complete) with tile
  // it + NST - 1, compute tile it.  A compression tile also stores its scores
  // (kScoreStores vector-memory operations, issued after the refill): those of
  // tile it-1 may still be in flight at the wait.  At it = 0 every load is
  // complete already (the wait for Q).
  constexpr int kScoreStores = 4;
  for (int it = 0; it < nt; ++it) {
    if (it + NST - 2 < nt) {
      if (branch == 0)
        vm_wait<(NST - 2) * LT + kScoreStores>();
      else
        vm_wait<(NST - 2) * LT>();
    } else {
      vm_wait<0>();
    }
    __syncthreads();
    if (it + NST - 1 < nt) request(it + NST - 1);
    int r0, lo, hi;
    tile_of(it, r0, lo, hi);
    dec_tile<T, D>(acc, m_, l_, qf, sK[it % NST], sV[it % NST], r0, lo, hi, a.sl2, lane, srow);
  }

  const float lt = l_ + __shfl_xor(l_, 32, kWave);
  if (n >= Gc) return;
  const int64_t pidx = ((int64_t)grp * nsp + split) * 32 + n;
  float* ml = (sel_phase ? a.p3_ml : a.p1_ml) + 2 * pidx;
  float* po = (sel_phase ? a.p3_o : a.p1_o) + pidx * D;
  if (h == 0) *reinterpret_cast<float2*>(ml) = make_float2(m_, lt);
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * dt + 8 * g4 + 4 * h;
      if (D % 32 == 0 || d < D)
        *reinterpret_cast<f32x4*>(po + d) =
            (f32x4){acc[dt][4 * g4], acc[dt][4 * g4 + 1], acc[dt][4 * g4 + 2], acc[dt][4 * g4 + 3]};
    }
}

__device__ __forceinline__ float dec_wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}
__device__ __forceinline__ float dec_wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// (max, sum) of the split partials p0 + 32 k, k < ns (float2 at ml + 2 p):
// the lanes take the splits, then the wave combines them.  ns > 0.
__device__ __forceinline__ void dec_merge_ml(const float* ml, int64_t p0, int ns, int lane, float& M, float& S) {
  float m = kDecNegInf, l = 0.0f;
  for (int k = lane; k < ns; k += kWave) {
    const float2 v = *reinterpret_cast<const float2*>(ml + 2 * (p0 + 32 * (int64_t)k));
    const float mn = fmaxf(m, v.x);   // split maxima are finite, so mn is
    l = l * fast_exp2(m - mn) + v.y * fast_exp2(v.x - mn);
    m = mn;
  }
  M = dec_wave_max(m);
  S = dec_wave_sum(l * fast_exp2(m - M));   // lanes without a split: exp2(-inf) = 0
}

constexpr int kDecTokPerWG = 1024;      // pooled tokens per token-sum workgroup (256 threads x 4)
constexpr int kDecTopnThreads = 1024;   // top-n workgroup: candidate blocks tid + 1024 k
constexpr int kDecKeysPerThread = kDecMaxCand / kDecTopnThreads;
constexpr int kDecMaxSel = 64;          // picks per query (one lane each in the final sort)

// Every head's log-sum-exp (log2 units) over the compression splits of one
// (b, hkv), into lse2[G]: threads 0 .. 255 of the workgroup, a wave per head
// (lph lanes per head, heads side by side), lanes over the splits, then
// combined across the head's lanes.
__device__ __forceinline__ void dec_head_lse2(const DecGeom& g, const float* __restrict__ p1_ml, int bh,
                                              int ncs_len, float* lse2, int tid) {
  const int nsp = g.ncs + g.nws;
  int lph = 64;   // lanes per head: a power of two <= 64
  while (lph > 1 && lph * g.G > 256) lph >>= 1;
  for (int h0 = 0; h0 < g.G; h0 += 256 / lph) {
    const int hd = h0 + tid / lph, sub = tid % lph;
    const int hs = hd < g.G ? hd : g.G - 1;
    const float* ml = p1_ml + 2 * (((int64_t)(bh * g.NHC + hs / 32) * nsp) * 32 + hs % 32);
    float m = kDecNegInf, l = 0.0f;
    for (int k0 = sub; k0 < ncs_len; k0 += 4 * lph) {
      float2 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + u * lph < ncs_len) v[u] = *reinterpret_cast<const float2*>(ml + 64 * (int64_t)(k0 + u * lph));
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + u * lph < ncs_len) {
          const float mn = fmaxf(m, v[u].x);   // split maxima are finite
          l = l * fast_exp2(m - mn) + v[u].y * fast_exp2(v[u].x - mn);
          m = mn;
        }
    }
    float M = m;
    for (int off = 1; off < lph; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, kWave));
    float S = l * fast_exp2(m - M);   // lanes without a split: exp2(-inf) = 0
    for (int off = 1; off < lph; off <<= 1) S += __shfl_xor(S, off, kWave);
    if (sub == 0 && hd < g.G) lse2[hd] = M + __log2f(S);
  }
}

// p_cmp of pooled tokens i4 .. i4 + 3 of one (b, hkv) summed over the group's
// heads (each head's four scores in one 16-byte load; heads 0-7, then 8-15,
// of each 16-head chunk, as the prefill importance kernel sums them)
__device__ __forceinline__ void dec_token_sums4(const DecGeom& g, const float* __restrict__ s_cmp, int bh, int i4,
                                                const float* lse2, float sl2, float (&v)[4]) {
  const float* sc = s_cmp + (int64_t)bh * g.G * g.NcapP;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = 0.0f;
  for (int c0 = 0; c0 < g.G; c0 += 16) {
    f32x4 x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)   // past nvis (inside the row pitch) the values are never used
      x[j] = c0 + j < g.G ? *reinterpret_cast<const f32x4*>(sc + (int64_t)(c0 + j) * g.NcapP + i4)
                          : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float half[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int hd = c0 + 8 * hh + j;
          if (hd < g.G) sum += fast_exp2(x[8 * hh + j][e] * sl2 - lse2[hd]);
        }
        half[hh] = sum;
      }
      v[e] = c0 == 0 ? half[0] + half[1] : v[e] + (half[0] + half[1]);
    }
  }
}

// p_cmp summed over the group's heads for 1024 pooled tokens of one (b, hkv)
// (dec_head_lse2, then four tokens per thread: dec_token_sums4).
template <typename T>
__global__ __launch_bounds__(256) void k_dec_toksum(const DecArgs<T> a, int nch) {
  extern __shared__ __align__(16) float lse2[];
  const DecGeom& g = a.g;
  const int tid = threadIdx.x;
  const int bh = blockIdx.x / nch, ch = blockIdx.x % nch, b = bh / g.Hkv;
  const DecLen L = dec_len(a.lens[b], g);
  const int i0 = ch * kDecTokPerWG;
  if (i0 >= L.nvis) return;
  dec_head_lse2(g, a.p1_ml, bh, dec_cmp_splits(L, g), lse2, tid);
  __syncthreads();
  const int i4 = i0 + 4 * tid;
  if (i4 >= L.nvis) return;
  float v[4];
  dec_token_sums4(g, a.s_cmp, bh, i4, lse2, a.sl2, v);
  float* dst = a.tok + (int64_t)bh * g.NcapP + i4;
  if (i4 + 3 < L.nvis) {
    *reinterpret_cast<f32x4*>(dst) = (f32x4){v[0], v[1], v[2], v[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i4 + e < L.nvis) dst[e] = v[e];
  }
}

// Block importance and the top S of one (b, hkv).  Candidate block j (thread
// j % 1024, register j / 1024) folds the token sums whose span meets it,
// tokens ascending, weighted by overlap / cd.  Its key is (order key of the
// score: +inf forced, -FLT_MAX incomplete) << 32 | ~j, unique, so the top S
// keys are the highest scores with ties to the lower block.  They are found
// by radix selection (eight 8-bit digits from the top: a histogram of the
// keys that match the digits fixed so far, and the digit at which the count
// from the top reaches the picks still needed), gathered, and sorted
// descending across the lanes of one wave.  FUSE: the workgroup forms the
// token sums itself (k_dec_toksum's arithmetic, so the same bits) instead of
// reading them, one launch and one round trip less when the pooled sequence
// is short.
template <bool FUSE>
__global__ __launch_bounds__(kDecTopnThreads) void k_dec_topn(const int32_t* __restrict__ lens,
                                                             const float* __restrict__ tok,
                                                             int32_t* __restrict__ idx, float* __restrict__ scores,
                                                             int ncand_cap, DecGeom g, float rcd,
                                                             const float* __restrict__ p1_ml,
                                                             const float* __restrict__ s_cmp, float sl2) {
  __shared__ uint32_t hist[2][256];
  __shared__ uint64_t ctl_prefix;
  __shared__ int ctl_need;
  __shared__ uint64_t picked[kDecMaxSel];
  __shared__ int npicked;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int bh = blockIdx.x, b = bh / g.Hkv;
  const DecLen L = dec_len(lens[b], g);
  int32_t* orow = idx + (int64_t)bh * g.n_sel;
  extern __shared__ __align__(16) float tk[];   // token sums [NcapP] (FUSE: then lse2 [G])
  if (tid < 256) hist[0][tid] = 0;
  if (tid == 0) npicked = 0;
  if constexpr (FUSE) {
    float* lse2 = tk + g.NcapP;
    if (L.nvis > 0) {   // uniform
      if (tid < 256) dec_head_lse2(g, p1_ml, bh, dec_cmp_splits(L, g), lse2, tid);
      __syncthreads();
      for (int i4 = 4 * tid; i4 < L.nvis; i4 += 4 * kDecTopnThreads) {
        float v[4];
        dec_token_sums4(g, s_cmp, bh, i4, lse2, sl2, v);
        *reinterpret_cast<f32x4*>(tk + i4) = (f32x4){v[0], v[1], v[2], v[3]};   // inside the row pitch
      }
    }
  } else {
    const float* src = tok + (int64_t)bh * g.NcapP;
    for (int i = 4 * tid; i < L.nvis; i += 4 * kDecTopnThreads)   // rows are 32-float aligned
      *reinterpret_cast<f32x4*>(tk + i) = *reinterpret_cast<const f32x4*>(src + i);
  }
  __syncthreads();
  const int tb = L.t / g.ls;
  uint64_t key[kDecKeysPerThread];
#pragma unroll
  for (int k = 0; k < kDecKeysPerThread; ++k) {
    const int j = tid + kDecTopnThreads * k;
    key[k] = 0;
    if (j < L.ncand) {
      const int lo = j * g.ls, hi = (j + 1) * g.ls;
      const int ia = lo - g.cl + 1 <= 0 ? 0 : (lo - g.cl + 1 + g.cd - 1) / g.cd;
      int ib = (hi - 1) / g.cd;
      ib = ib < L.nvis - 1 ? ib : L.nvis - 1;
      float sum = 0.0f;
      for (int i = ia; i <= ib; ++i) {
        const int x0 = i * g.cd > lo ? i * g.cd : lo;
        const int x1 = i * g.cd + g.cl < hi ? i * g.cd + g.cl : hi;
        if (x1 > x0) sum += tk[i] * ((float)(x1 - x0) * rcd);
      }
      if (scores != nullptr) scores[(int64_t)bh * ncand_cap + j] = sum;
      const bool valid = hi - 1 <= L.t;
      const bool forced = (g.force_init && j == 0) || (j <= tb && j > tb - g.n_local);
      const float sc = forced ? __builtin_inff() : (valid ? sum : -3.4028234663852886e38f);
      key[k] = ((uint64_t)order_key(sc) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)j);
    }
  }
  const int S = L.S;
  if (S > 0) {   // uniform: every thread of the workgroup sees the same L
    uint64_t prefix = 0, mask = 0;
    int need = S;
    for (int p = 0; p < 8; ++p) {
      const int shift = 56 - 8 * p;
      uint32_t* h = hist[p & 1];
      if (tid < 256) hist[(p + 1) & 1][tid] = 0;   // the other buffer: last read before the previous barrier
      __syncthreads();
#pragma unroll
      for (int k = 0; k < kDecKeysPerThread; ++k)
        if (key[k] != 0 && (key[k] & mask) == prefix) atomicAdd(&h[(uint32_t)(key[k] >> shift) & 255u], 1u);
      __syncthreads();
      if (w == 0) {
        // lane l holds digits 255 - 4l .. 252 - 4l (highest first)
        uint32_t c[4], tot = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) tot += (c[i] = h[255 - 4 * lane - i]);
        uint32_t incl = tot;   // inclusive scan over the lanes, from lane 0
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
          const uint32_t y = (uint32_t)__shfl_up((int)incl, off, kWave);
          incl += lane >= off ? y : 0u;
        }
        uint32_t run = incl - tot;   // keys above this lane's digits
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (run < (uint32_t)need && run + c[i] >= (uint32_t)need) {
            ctl_prefix = prefix | ((uint64_t)(255 - 4 * lane - i) << shift);
            // the whole bucket is picked: the remaining digits can stay 0
            ctl_need = run + c[i] == (uint32_t)need ? 0 : need - (int)run;
          }
          run += c[i];
        }
      }
      __syncthreads();
      prefix = ctl_prefix;
      need = ctl_need;
      mask |= (uint64_t)255 << shift;
      if (need == 0) break;
    }
    // exactly S keys are >= prefix (the S-th highest key, or the lowest
    // possible key of a bucket that is picked whole)
#pragma unroll
    for (int k = 0; k < kDecKeysPerThread; ++k)
      if (key[k] != 0 && key[k] >= prefix) picked[atomicAdd(&npicked, 1)] = key[k];
    __syncthreads();
    if (w == 0) {
      uint64_t x = lane < S ? picked[lane] : 0;
      // bitonic sort, descending across the 64 lanes
      for (int k = 2; k <= kWave; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
          const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, j, kWave);
          const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), j, kWave);
          const uint64_t y = ((uint64_t)hi << 32) | lo;
          const bool desc = (lane & k) == 0, low = (lane & j) == 0;
          x = (low == desc) ? (y > x ? y : x) : (y < x ? y : x);
        }
      if (lane < S) orow[lane] = (int32_t)(0xFFFFFFFFu - (uint32_t)x);
    }
  }
  for (int s = S + tid; s < g.n_sel; s += kDecTopnThreads) orow[s] = -1;
}

// One workgroup per query head, one wave per branch (gate order:
// compression, selection, window): the branch's (max, sum) over its splits,
// then its output, the lanes split 8 ways over the splits and 8 ways over
// 4-element column runs (16-byte loads), summed across the split groups at
// the end; the gated sum adds the branches in gate order.
template <typename T, int D>
__global__ __launch_bounds__(192) void k_dec_merge(const DecArgs<T> a) {
  const DecGeom& g = a.g;
  __shared__ __align__(16) float so[3][D];
  const int c = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x;   // b * Hq + hq
  const int b = (int)(row / g.Hq), hq = (int)(row % g.Hq);
  const int hkv = hq / g.G, hd = hq % g.G;
  const int grp = (b * g.Hkv + hkv) * g.NHC + hd / 32, col = hd % 32;
  const DecLen L = dec_len(a.lens[b], g);
  const int64_t nrow = (int64_t)g.B * g.Hq;
  constexpr int RUNS = D / 4 < 8 ? D / 4 : 8;      // lanes per split over the columns
  constexpr int EPL = D / (4 * RUNS);              // 4-element runs per lane
  constexpr int UNR = 4;                           // splits per group whose loads go out together
  const int sg = lane / RUNS, dl = lane % RUNS;    // split group, column lane
  constexpr int NSG = kWave / RUNS;
  const float* ml;
  const float* po;
  int nsp, s0, ns;
  if (c == 1) {
    ml = a.p3_ml, po = a.p3_o, nsp = g.nss, s0 = 0, ns = L.t < 0 ? 0 : dec_sel_splits(L, g);
  } else {
    ml = a.p1_ml, po = a.p1_o, nsp = g.ncs + g.nws;
    s0 = c == 0 ? 0 : g.ncs;
    ns = L.t < 0 ? 0 : (c == 0 ? dec_cmp_splits(L, g) : dec_win_splits(L, g));
  }
  const int64_t p0 = ((int64_t)grp * nsp + s0) * 32 + col;
  // each split group keeps a running (max, sum, output) over its splits
  // (loads of UNR splits in flight), then the groups are rescaled to the
  // common maximum and summed
  float M = kDecNegInf, S = 0.0f;
  f32x4 o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  if (ns > 0) {
    for (int k0 = 0; k0 < ns; k0 += NSG * UNR) {
      float2 mv[UNR];
      f32x4 ov[UNR][EPL];
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int k = k0 + NSG * u + sg;
        if (k < ns) {   // lanes past the last split issue no load
          const int64_t p = p0 + 32 * (int64_t)k;
          mv[u] = *reinterpret_cast<const float2*>(ml + 2 * p);
#pragma unroll
          for (int e = 0; e < EPL; ++e)
            ov[u][e] = *reinterpret_cast<const f32x4*>(po + p * D + 4 * (dl + RUNS * e));
        }
      }
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        if (k0 + NSG * u + sg < ns) {
          const float mn = fmaxf(M, mv[u].x);   // split maxima are finite
          const float a0 = fast_exp2(M - mn), a1 = fast_exp2(mv[u].x - mn);
          S = S * a0 + mv[u].y * a1;
#pragma unroll
          for (int e = 0; e < EPL; ++e) o[e] = o[e] * a0 + ov[u][e] * a1;
          M = mn;
        }
      }
    }
    float Mw = M;
#pragma unroll
    for (int off = RUNS; off < kWave; off <<= 1) Mw = fmaxf(Mw, __shfl_xor(Mw, off, kWave));
    const float r = fast_exp2(M - Mw);   // groups without a split: exp2(-inf) = 0
    S *= r;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] *= r;
#pragma unroll
    for (int off = RUNS; off < kWave; off <<= 1) {
      S += __shfl_xor(S, off, kWave);
#pragma unroll
      for (int e = 0; e < EPL; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[e][i] += __shfl_xor(o[e][i], off, kWave);
    }
    M = Mw;
  }
  const float inv = S > 0.0f ? 1.0f / S : 0.0f;
  if (sg == 0) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int d = 4 * (dl + RUNS * e);
      const f32x4 v = o[e] * inv;
      *reinterpret_cast<f32x4*>(&so[c][d]) = v;
      if (a.o_branch != nullptr) *reinterpret_cast<f32x4*>(a.o_branch + ((int64_t)c * nrow + row) * D + d) = v;
    }
  }
  if (a.lse_branch != nullptr && lane == 0)
    a.lse_branch[(int64_t)c * nrow + row] = S > 0.0f ? (M + __log2f(S)) * kLn2 : kLseEmpty;
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 192) {
    float r = 0.0f;
#pragma unroll
    for (int cc = 0; cc < 3; ++cc) {
      const float gl = to_f32(a.gate[row * 3 + cc]);
      r += (1.0f / (1.0f + __expf(-gl))) * so[cc][d];
    }
    a.out[row * D + d] = from_f32<T>(r);
  }
}

// Append one token to the caches of every (b, hkv): the six branch K/V rows
// at position lens_in[b], and -- when the new length completes a pooled
// span -- the pooled compression token, summed in the order of the pooling
// kernel (rows ascending, then * 1/cl) so the cache holds exactly what
// nsa_pool_fwd writes.  Sequences whose cache is full are left unchanged.
template <typename T>
struct DecCaches {
  T* kv[6];            // kc vc ks vs kw vw  [B][Hkv][Tcap][D]
  const T* nw[6];      // new rows           [B][Hkv][D]
  T* kcmp;             // [B][Hkv][Ncap][D]
  T* vcmp;
};

template <typename T>
__global__ __launch_bounds__(256) void k_dec_append(const DecCaches<T> c, const int32_t* __restrict__ lens_in,
                                                    int32_t* __restrict__ lens_out, int Hkv, int D, int Tcap,
                                                    int Ncap, int cl, int cd) {
  const int bh = blockIdx.x, b = bh / Hkv, tid = threadIdx.x;
  const int pos = lens_in[b];
  const bool room = pos >= 0 && pos < Tcap;
  const int dc = D / 8;
  if (room) {
    for (int e = tid; e < 6 * dc; e += 256) {
      const int which = e / dc, ch = e % dc;
      Frag<T> f;
      f.load(c.nw[which] + (int64_t)bh * D + 8 * ch);
      f.store(c.kv[which] + ((int64_t)bh * Tcap + pos) * D + 8 * ch);
    }
    const int Lp = pos + 1;
    if (Lp >= cl && (Lp - cl) % cd == 0 && (Lp - cl) / cd < Ncap) {
      const int i = (Lp - cl) / cd;
      const float inv = 1.0f / (float)cl;
      for (int e = tid; e < 2 * dc; e += 256) {
        const int kv = e / dc, ch = e % dc;   // 0: keys (kc), 1: values (vc)
        const T* src = c.kv[kv] + ((int64_t)bh * Tcap + (int64_t)i * cd) * D + 8 * ch;
        float s[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] = 0.0f;
        for (int k = 0; k < cl; ++k) {
          Frag<T> f;
          f.load(k == cl - 1 ? c.nw[kv] + (int64_t)bh * D + 8 * ch : src + (int64_t)k * D);
#pragma unroll
          for (int j = 0; j < 8; ++j) s[j] += to_f32(f.elem(j));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] *= inv;
        Frag<T> o;
        o.set(s);
        o.store((kv == 0 ? c.kcmp : c.vcmp) + ((int64_t)bh * Ncap + i) * D + 8 * ch);
      }
    }
  }
  if (bh % Hkv == 0 && tid == 0) lens_out[b] = room ? pos + 1 : pos;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static inline size_t dec_align(size_t x) { return (x + 255) & ~(size_t)255; }

struct DecPlan {
  DecGeom g;
  size_t off_p1_ml, off_p1_o, off_p3_ml, off_p3_o, off_s, off_tok, total;
  int ncand_cap;
};

static int dec_plan(DecPlan& P, int B, int Hq, int Hkv, int D, int Tcap, int Ncap, int cl, int cd, int ls, int n_sel,
                    int window, int force_init, int n_local) {
  NSA_CHECK(B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(cl >= 1 && cd >= 1 && ls >= 1 && n_sel >= 0 && window >= 1 && n_local >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(n_sel <= kDecMaxSel && Hq / Hkv <= 1024, NSA_ERR_SHAPE);
  NSA_CHECK(Tcap >= 1 && Ncap >= 0, NSA_ERR_SHAPE);
  const int n_need = Tcap >= cl ? (Tcap - cl) / cd + 1 : 0;
  NSA_CHECK(Ncap >= n_need, NSA_ERR_SHAPE);
  const int ncand_cap = (Tcap - 1) / ls + 1;
  NSA_CHECK(ncand_cap <= kDecMaxCand, NSA_ERR_SHAPE);
  DecGeom& g = P.g;
  g.B = B, g.Hq = Hq, g.Hkv = Hkv, g.G = Hq / Hkv, g.NHC = (g.G + 31) / 32;
  g.Tcap = Tcap, g.Ncap = Ncap, g.NcapP = ((n_need > 0 ? n_need : 1) + 31) / 32 * 32;
  g.cl = cl, g.cd = cd, g.ls = ls, g.tpb = (ls + 31) / 32;
  g.n_sel = n_sel, g.window = window, g.force_init = force_init ? 1 : 0, g.n_local = n_local;
  const int nwt_max_w = (window + 30) / 32 + 1, nwt_max_t = (Tcap + 31) / 32;
  const int nwt_max = nwt_max_w < nwt_max_t ? nwt_max_w : nwt_max_t;
  const int smax = n_sel < ncand_cap ? n_sel : ncand_cap;
  // tiles per split: the most (up to 8 compression, 4 window / selection)
  // that still give each phase about a thousand single-wave workgroups, so
  // small batches spread over the CUs and large ones keep the partials few
  const int64_t ng = (int64_t)B * Hkv * ((Hq / Hkv + 31) / 32);
  auto per_split = [&](int tiles, int most, int64_t want) {
    int t = most;
    while (t > 1 && ng * ((tiles + t - 1) / t) < want) t /= 2;
    return t;
  };
  const int ctiles = (n_need + 31) / 32, stiles = smax * ((ls + 31) / 32);
  g.ct = per_split(ctiles, kDecMaxTiles, 1024);
  g.wt = per_split(nwt_max, 4, 256);
  g.st = per_split(stiles, 4, 1024);
  g.ncs = (ctiles + g.ct - 1) / g.ct;
  g.nws = (nwt_max + g.wt - 1) / g.wt;
  g.nss = (stiles + g.st - 1) / g.st;
  if (g.nss < 1) g.nss = 1;
  const size_t NG = (size_t)B * Hkv * g.NHC;
  const size_t n1 = NG * (g.ncs + g.nws) * 32, n3 = NG * g.nss * 32;
  P.off_p1_ml = 0;
  P.off_p1_o = dec_align(P.off_p1_ml + n1 * 2 * sizeof(float));
  P.off_p3_ml = dec_align(P.off_p1_o + n1 * D * sizeof(float));
  P.off_p3_o = dec_align(P.off_p3_ml + n3 * 2 * sizeof(float));
  P.off_s = dec_align(P.off_p3_o + n3 * D * sizeof(float));
  // the top-n workgroup stages one sequence's token sums in LDS
  NSA_CHECK((size_t)g.NcapP * sizeof(float) <= 128 * 1024, NSA_ERR_SHAPE);
  P.off_tok = dec_align(P.off_s + (size_t)B * Hkv * g.G * g.NcapP * sizeof(float));
  P.total = dec_align(P.off_tok + (size_t)B * Hkv * g.NcapP * sizeof(float));
  P.ncand_cap = ncand_cap;
  return NSA_OK;
}

template <typename T, int D>
static int dec_launch(const DecArgs<T>& a, const DecPlan& P, hipStream_t s) {
  // two stages (one tile in flight while the other computes): 32 KB of LDS
  // per bf16 D = 128 wave, five waves per CU -- measured 10% faster at 32
  // sequences x 32K than three stages at three waves per CU
  constexpr int NST = 2;
  const DecGeom& g = P.g;
  const int64_t NG = (int64_t)g.B * g.Hkv * g.NHC;
  const int64_t g1 = NG * (g.ncs + g.nws), g3 = NG * g.nss;
  NSA_CHECK(g1 < (1ll << 31) && g3 < (1ll << 31), NSA_ERR_SHAPE);
  if (g1 > 0) k_dec_part<T, D, NST><<<(unsigned)g1, 64, 0, s>>>(a, 0);
  const int nch = (g.NcapP + kDecTokPerWG - 1) / kDecTokPerWG;
  const int64_t gt = (int64_t)g.B * g.Hkv * nch;
  NSA_CHECK(gt < (1ll << 31), NSA_ERR_SHAPE);
  // short pooled sequences (two token-sum chunks at most): the top-n
  // workgroup forms the token sums itself
  const bool fuse = nch <= 2;
  if (g.ncs > 0 && !fuse) k_dec_toksum<T><<<(unsigned)gt, 256, sizeof(float) * g.G, s>>>(a, nch);
  const size_t topn_lds = sizeof(float) * (g.NcapP + (fuse ? g.G : 0));
  const void* topn = fuse ? (const void*)k_dec_topn<true> : (const void*)k_dec_topn<false>;
  if (topn_lds > 48 * 1024 &&
      hipFuncSetAttribute(topn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)topn_lds) != hipSuccess)
    return NSA_ERR_LAUNCH;
  auto topn_kern = fuse ? k_dec_topn<true> : k_dec_topn<false>;
  topn_kern<<<(unsigned)(g.B * g.Hkv), kDecTopnThreads, topn_lds, s>>>(
      a.lens, a.tok, a.idx, a.scores, a.ncand_cap, g, 1.0f / (float)g.cd, a.p1_ml, a.s_cmp, a.sl2);
  k_dec_part<T, D, NST><<<(unsigned)g3, 64, 0, s>>>(a, 1);
  const int64_t rows = (int64_t)g.B * g.Hq;
  NSA_CHECK(rows < (1ll << 31), NSA_ERR_SHAPE);
  k_dec_merge<T, D><<<(unsigned)rows, 192, 0, s>>>(a);
  return nsa_launch_status();
}

}  // namespace nsa

using namespace nsa;

extern "C" {

size_t nsa_decode_workspace(int B, int Hq, int Hkv, int D, int Tcap, int Ncap, int cmp_block, int cmp_stride,
                            int sel_block, int n_sel, int window) {
  DecPlan P;
  if (dec_plan(P, B, Hq, Hkv, D, Tcap, Ncap, cmp_block, cmp_stride, sel_block, n_sel, window, 0, 0) != NSA_OK)
    return 0;
  return P.total;
}

int nsa_decode_fwd(const void* q, const void* k_cmp, const void* v_cmp, const void* ks, const void* vs, const void* kw,
                   const void* vw, const void* gate, const int32_t* lens, void* out, int32_t* block_idx,
                   float* scores, float* o_branch, float* lse_branch, void* workspace, size_t workspace_bytes, int B,
                   int Hq, int Hkv, int D, int Tcap, int Ncap, int cmp_block, int cmp_stride, int sel_block,
                   int n_sel, int window, int force_init, int n_local, int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  DecPlan P;
  const int rc = dec_plan(P, B, Hq, Hkv, D, Tcap, Ncap, cmp_block, cmp_stride, sel_block, n_sel, window, force_init,
                          n_local);
  if (rc != NSA_OK) return rc;
  NSA_CHECK(q && ks && vs && kw && vw && gate && lens && out && block_idx, NSA_ERR_ARG);
  NSA_CHECK(P.g.ncs == 0 || (k_cmp && v_cmp), NSA_ERR_ARG);
  NSA_CHECK(workspace != nullptr && workspace_bytes >= P.total && ((uintptr_t)workspace & 255) == 0,
            NSA_ERR_WORKSPACE);
  char* ws = (char*)workspace;
  auto fill = [&](auto tag) -> int {
    using T = decltype(tag);
    DecArgs<T> a;
    a.q = (const T*)q, a.kcmp = (const T*)k_cmp, a.vcmp = (const T*)v_cmp, a.ks = (const T*)ks, a.vs = (const T*)vs;
    a.kw = (const T*)kw, a.vw = (const T*)vw, a.gate = (const T*)gate, a.lens = lens, a.out = (T*)out;
    a.idx = block_idx, a.scores = scores, a.o_branch = o_branch, a.lse_branch = lse_branch;
    a.p1_ml = (float*)(ws + P.off_p1_ml), a.p1_o = (float*)(ws + P.off_p1_o);
    a.p3_ml = (float*)(ws + P.off_p3_ml), a.p3_o = (float*)(ws + P.off_p3_o);
    a.s_cmp = (float*)(ws + P.off_s);
    a.tok = (float*)(ws + P.off_tok);
    a.ncand_cap = P.ncand_cap;
    a.sl2 = (1.0f / sqrtf((float)D)) * kLog2e;
    a.g = P.g;
    hipStream_t s = (hipStream_t)stream;
    switch (D) {
      case 16: return dec_launch<T, 16>(a, P, s);
      case 32: return dec_launch<T, 32>(a, P, s);
      case 64: return dec_launch<T, 64>(a, P, s);
      case 128: return dec_launch<T, 128>(a, P, s);
      default: return NSA_ERR_SHAPE;
    }
  };
  return dtype == NSA_BF16 ? fill(bf16{}) : fill(float{});
}

int nsa_decode_append(void* kc, void* vc, void* ks, void* vs, void* kw, void* vw, void* k_cmp, void* v_cmp,
                      const void* kc_new, const void* vc_new, const void* ks_new, const void* vs_new,
                      const void* kw_new, const void* vw_new, const int32_t* lens_in, int32_t* lens_out, int B,
                      int Hkv, int D, int Tcap, int Ncap, int cmp_block, int cmp_stride, int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(B > 0 && Hkv > 0 && Tcap >= 1 && Ncap >= 0 && cmp_block >= 1 && cmp_stride >= 1, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(kc && vc && ks && vs && kw && vw && kc_new && vc_new && ks_new && vs_new && kw_new && vw_new, NSA_ERR_ARG);
  NSA_CHECK(lens_in && lens_out && (const void*)lens_in != (const void*)lens_out, NSA_ERR_ARG);
  NSA_CHECK(Ncap == 0 || (k_cmp && v_cmp), NSA_ERR_ARG);
  hipStream_t s = (hipStream_t)stream;
  auto go = [&](auto tag) {
    using T = decltype(tag);
    DecCaches<T> c;
    void* dst[6] = {kc, vc, ks, vs, kw, vw};
    const void* src[6] = {kc_new, vc_new, ks_new, vs_new, kw_new, vw_new};
    for (int i = 0; i < 6; ++i) c.kv[i] = (T*)dst[i], c.nw[i] = (const T*)src[i];
    c.kcmp = (T*)k_cmp, c.vcmp = (T*)v_cmp;
    k_dec_append<T><<<(unsigned)(B * Hkv), 256, 0, s>>>(c, lens_in, lens_out, Hkv, D, Tcap, Ncap, cmp_block,
                                                         cmp_stride);
  };
  if (dtype == NSA_BF16)
    go(bf16{});
  else
    go(float{});
  return nsa_launch_status();
}

}  // extern "C"
