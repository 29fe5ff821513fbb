// Key-side NSA backward: dK/dV of the range branches (window, compression)
// and of the selection branch (block-outer over the block -> query CSR),
// LDS-tiled on 32x32 MFMAs.
//
// A wave owns 32 keys: their K and V fragments stay in registers and their
// dK^T / dV^T accumulate in registers for the whole walk.  The queries that
// see those keys stream through LDS two at a time (32 rows = two queries x 16
// heads of a head chunk; groups of fewer heads fill a tile with more queries:
// GroupTiles for the selection, FlatReq for the range branches): row tiles of
// Q and dO (direct global -> LDS loads,
// kKvStages deep) and per-row statistics c = lse*log2(e) - log2(rowscale)
// and delta, shared by the workgroup's waves.
//   S = Q K^T, dP = dO V^T                     (rows on M, keys on N)
//   P = exp2(S*scale*log2(e) - c), dS = P (dP - delta)
//   dV^T += dO^T P,  dK^T += Q^T dS             (P / dS straight from the accumulators)
// Q / dO are read through perm32 for the first pair of products and
// transposed (ds_read_b64_tr_b16) for the second, so one copy of each tile
// serves both and the S / dP accumulators line up with the operand slots.
// Tiles whose two queries see all 32 keys of a wave skip the per-element mask.
//
//   * window      : a workgroup owns 32*NW keys and walks queries [k0, k0 + 32 NW + w - 2].
//   * compression : same, over query chunks of kCmpChunk; chunks merge with
//                   float atomics; the key blocks of one chunk share an XCD.
//   For 16-bit operands both run the role-split walk (kv_walk's work on two
//   waves per 32 keys, two waves per SIMD; below).
//   * selection   : work items (block, chunk of its CSR query list) built by
//                   k_sel_items; a persistent grid drains them; chunks merge with atomics.
#include <atomic>
#include <mutex>

#include "nsa_launch.h"
#include "nsa_items.h"
#include "nsa_tile32.h"

namespace nsa {

constexpr int kKvStages = 4;   // query tiles in flight per workgroup (3 loads ahead)

// Row offset of rows that do not exist (a missing second query, heads past
// the group): exp2(s - inf) = 0 removes them from every product.
__device__ const float kAbsentRow = __builtin_inff();

template <typename T, int D> struct KvStage {
  using C = Tile32<T, D>;
  T qr[C::ROW_ELEMS];    // Q rows   [32][D]; row r = query (r >> 4), head (r & 15)
  T dr[C::ROW_ELEMS];    // dO rows  [32][D]
  float c[32], dot[32];  // filled by one 64-lane load: c then dot
  int meta[4];           // tA, tB, sA, sB of the tile (tB = -1: none)
};

// Read-only inputs of the query side.  Q and dO are either [B, Hq, T, D]
// (hs = T D, ts = D) or packed per query [B, Hkv, T, G, D] (hs = D, ts = G D):
// element (b, hkv, head g of the group, query t) is at
// (b Hkv + hkv) G T D + g hs + t ts either way.  The row statistics c and dot
// follow the same layout without D: [B, Hq, T] (sh = T, st = 1) or packed
// [B, Hkv, T, G] (sh = 1, st = G), so that a tile of two queries reads them
// from two 64-byte runs instead of one cache line per row.
template <typename T> struct QSide {
  const T* q;
  const T* dout;
  const float* c;     // per-row exponent offset lse*log2(e) - log2(rowscale)
  const float* dot;
  int Hq, Hkv, G, NHC, T_;
  int64_t hs, ts;     // element strides between heads of a group / queries
  int sh, st;         // the same for the row statistics
};

// vector-memory loads one wave issues per query tile
template <typename T, int D, int NTH>
constexpr int kv_tile_loads() {
  return 2 * dma_uniform_loads<NTH, Tile32<T, D>::ROW_CHUNKS>() + 1;
}

// Issues the loads of one 2-query row tile into a stage: both operand tiles
// and the row statistics go straight to LDS, and the tile's query / slot ids
// are written for the consumer.  Rows that do not exist (heads past the
// group, a missing second query) read finite operand rows of a real row and
// the row offset +inf, so their P and dS are exactly 0.
//
// Everything that depends only on the lane and the head chunk is prepared
// once per head chunk (prepare()): each load's 32-bit byte offset below the
// tile's first row, whether its row is query B's, the chunk's element offset
// and this lane's statistics row.  Per tile, the query ids are made
// wave-uniform, the operand base is scalar arithmetic, and each load adds
// query B's row distance to its lane's offset when its rows are B's -- a
// wave-uniform choice whenever a wave's 64 chunks never straddle the two
// queries' halves of the tile (16 rows a multiple of 64 chunks).
template <typename T, int D, int NTH> struct KvIssuer {
  using C = Tile32<T, D>;
  static constexpr int LPT = dma_uniform_loads<NTH, C::ROW_CHUNKS>();   // loads per operand tile
  static constexpr bool UNI = (16 * C::RCH) % 64 == 0;
  uint32_t off[LPT];   // (head * hs + column) * sizeof(T) of this lane's chunk of load j
  uint32_t qsel;       // bit j: load j's row belongs to query B (per lane; unused when UNI)
  int64_t qbase;       // element offset of the head chunk's first head, query 0
  const float* sp;     // statistics row of this lane at query 0 (c for lanes < 32, delta above)
  int sbit;            // stats: this lane's row belongs to query B
  int sreal;           // stats: the head exists

  // first physical chunk of load j of wave w (wave-uniform)
  static __device__ __forceinline__ int first_chunk(int j, int w) {
    return (int)((uint32_t)(j * NTH + 64 * w) % (uint32_t)C::ROW_CHUNKS);
  }

  __device__ __forceinline__ void prepare(const QSide<T>& x, int b, int hkv, int hc, int tid) {
    const int grem = x.G - hc * 16;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    qsel = 0;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int r, cc;
      row_chunk<T, D>(first_chunk(j, w) + lane, r, cc);
      const int hd = (r & 15) < grem ? (r & 15) : grem - 1;
      off[j] = (uint32_t)(((uint64_t)hd * x.hs + cc * C::EPC) * sizeof(T));
      qsel |= (uint32_t)(r >> 4) << j;
    }
    qbase = ((int64_t)b * x.Hkv + hkv) * x.G * x.T_ * D + hc * 16 * x.hs;
    const int r = lane & 31;
    sbit = r >> 4;
    const int shead = (r & 15) < grem ? (r & 15) : grem - 1;
    sreal = (r & 15) < grem;
    const int64_t row0 = ((int64_t)b * x.Hkv + hkv) * x.G * x.T_ + (int64_t)(hc * 16 + shead) * x.sh;
    sp = (lane < 32 ? x.c : x.dot) + row0;
  }

  __device__ __forceinline__ void issue(KvStage<T, D>& s, const QSide<T>& x, int tA, int tB, int sA, int sB,
                                        int tid) const {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    tA = __builtin_amdgcn_readfirstlane(tA);
    tB = __builtin_amdgcn_readfirstlane(tB);
    const int tBq = tB >= 0 ? tB : tA;   // a missing second query re-reads the first
    // rows addressed upward from the lower query (whatever the entries' order)
    const PairRows pr = pair_rows(tA, tB, (uint32_t)(x.ts * sizeof(T)));
    const int64_t qoff = qbase + (int64_t)pr.t0 * x.ts;
    const T* qa = x.q + qoff;
    const T* da = x.dout + qoff;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int first = first_chunk(j, w);
      const bool rowB = UNI ? first / C::RCH >= 16 : ((qsel >> j) & 1u) != 0;
      const uint32_t v = off[j] + (rowB ? pr.dB : pr.dA);
      lds_dma16_sbase(qa, v, (char*)s.qr + 16 * first);
      lds_dma16_sbase(da, v, (char*)s.dr + 16 * first);
    }
    {
      // lanes 0-31: c of row lane, lanes 32-63: delta of row lane - 32
      const bool real = lane >= 32 || (sreal && (!sbit || tB >= 0));
      lds_dma4(real ? sp + (int64_t)(sbit ? tBq : tA) * x.st : &kAbsentRow, s.c);
    }
    if (tid == 0) {
      s.meta[0] = tA;
      s.meta[1] = tB;
      s.meta[2] = sA;
      s.meta[3] = sB;
    }
  }
};

// Visibility of a lane's key to the rows of a tile, by accumulator register r
// of KeyAcc::front (register r of lane half h holds row acc_elem(h, r)).
// Two-query tiles: rows 0-15 are query A's, rows 16-31 query B's.
struct VisPair {
  bool a, b;
  __device__ __forceinline__ bool operator()(int r) const { return r < 8 ? a : b; }
};
// Any row layout: bit e of the row mask says whether row e sees the key,
// stored shifted right by 8 h so that register r tests bit 16 (r >> 3) + (r & 7).
struct VisBits {
  uint32_t bits;
  __device__ __forceinline__ bool operator()(int r) const { return (bits >> (16 * (r >> 3) + (r & 7))) & 1u; }
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
    // complete the loads here: the walk's loads are invisible to the
    // compiler, which would otherwise wait on these inside the loop -- with
    // counts that also drain the walk's tiles in flight
#pragma unroll
    for (int s = 0; s < C::KS; ++s) settle(kf[s]), settle(vf[s]);
  }

  // Q / dO fragments of one tile (row operands of S and dP, read through perm32)
  struct Rows {
    Frag<T> qa[C::KS], da[C::KS];
  };
  __device__ __forceinline__ static void read_rows(Rows& q, const KvStage<T, D>& s, int lane) {
    const int h = lane >> 5, n = lane & 31;
#pragma unroll
    for (int k = 0; k < C::KS; ++k) {
      lds_row_frag<T, D>(q.qa[k], s.qr, n, h, k);
      lds_row_frag<T, D>(q.da[k], s.dr, n, h, k);
    }
  }

  // First half of a tile: S and dP from the row fragments read earlier, the
  // transposed fragments dO^T (ta) and Q^T (tb) read while those MFMAs run,
  // then P and dS packed as the operands of the second half.  With MASK,
  // vis(r) says whether this lane's key is visible to the row of accumulator
  // register r (VisPair, VisBits); without, every key is.
  template <bool MASK, typename Vis>
  __device__ __forceinline__ void front(const KvStage<T, D>& s, const Rows& q, const Vis& vis, float sl2,
                                        int lane, Frag<T> (&ta)[C::DT][2], Frag<T> (&tb)[C::DT][2],
                                        Frag<T> (&pf)[2], Frag<T> (&sf)[2]) {
    const int h = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        lds_tr_frag<T, D>(ta[dt][k], s.dr, dt, lane, k);
        lds_tr_frag<T, D>(tb[dt][k], s.qr, dt, lane, k);
      }
    f32x16 sacc = zero16(), pacc = zero16();
#pragma unroll
    for (int k = 0; k < C::KS; ++k) {
      mma32(sacc, q.qa[k], kf[k]);
      mma32(pacc, q.da[k], vf[k]);
    }
    if constexpr (sizeof(T) == 2) {
      // one MFMA, then its share of the transposed reads (left alone, the
      // scheduler issues each read right before its first use)
      constexpr int NTR = 2 * 2 * C::DT * 2;
      constexpr int PER = (NTR + 2 * C::KS - 1) / (2 * C::KS);
#pragma unroll
      for (int i = 0; i < 2 * C::KS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);
      }
    }
    float P[16], dS[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int e = acc_elem(h, r);
      float p = fast_exp2(sacc[r] * sl2 - s.c[e]);
      if (MASK) p = vis(r) ? p : 0.0f;
      P[r] = p;
      dS[r] = p * (pacc[r] - s.dot[e]);
    }
    pf[0].set(P);
    pf[1].set(P + 8);
    sf[0].set(dS);
    sf[1].set(dS + 8);
  }

  // Second half: dV^T += dO^T P, dK^T += Q^T dS (registers only)
  __device__ __forceinline__ void back(const Frag<T> (&ta)[C::DT][2], const Frag<T> (&tb)[C::DT][2],
                                       const Frag<T> (&pf)[2], const Frag<T> (&sf)[2]) {
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

// Row tiles of two queries x the 16 heads of a head chunk (KvIssuer), a tile
// source of kv_walk: the caller's qsrc(i, tA, tB, sA, sB) names tile i's
// queries and their block_idx slots (tB = -1: none) and vis(tA, tB, mask,
// visA, visB) fills a tile's mask flags for this wave (tB = -1: query B's rows
// are absent, whatever visB says).  The consumer reads the tile's queries back
// from the stage (the ids issue() wrote).
template <typename T, int D, int NTH, typename QSrc, typename Vis> struct PairTiles {
  struct Info {
    int tA, tB, sA, sB;
  };
  const QSide<T>& x;
  int b, hkv;
  QSrc qsrc;
  Vis visf;
  KvIssuer<T, D, NTH> iss;
  __device__ __forceinline__ void prepare(int hc, int tid) { iss.prepare(x, b, hkv, hc, tid); }
  __device__ __forceinline__ void issue(KvStage<T, D>& s, int ti, int tid) {
    int tA, tB, sA, sB;
    qsrc(ti, tA, tB, sA, sB);
    iss.issue(s, x, tA, tB, sA, sB, tid);
  }
  __device__ __forceinline__ Info info(const KvStage<T, D>& s, int) const {
    return Info{__builtin_amdgcn_readfirstlane(s.meta[0]), __builtin_amdgcn_readfirstlane(s.meta[1]),
                __builtin_amdgcn_readfirstlane(s.meta[2]), __builtin_amdgcn_readfirstlane(s.meta[3])};
  }
  __device__ __forceinline__ VisPair vis(const Info& i, bool& mask) const {
    VisPair v;
    visf(i.tA, i.tB, mask, v.a, v.b);
    return v;
  }
};
template <typename T, int D, int NTH, typename QSrc, typename Vis>
__device__ __forceinline__ PairTiles<T, D, NTH, QSrc, Vis> pair_tiles(const QSide<T>& x, int b, int hkv, QSrc qsrc,
                                                                     Vis vis) {
  return PairTiles<T, D, NTH, QSrc, Vis>{x, b, hkv, qsrc, vis, {}};
}

// Row tiles of QPT = floor(32 / G) CSR entries of a selection work item, for
// GQA groups of G <= 10 heads (a tile of two queries would leave 32 - 2 G of
// its rows empty): rows q G .. q G + G - 1 are entry q's heads, rows from
// QPT G on are absent.  Q / dO and the row statistics are in the packed
// per-query layout, so row (t, g) of the group is row t G + g from the
// group's base.  A lane's loads are prepared once (the entry q and head g of
// its chunks' rows); per tile it reads its entries' queries from the item's
// entries in LDS and adds t G D elements to its offsets.  Absent rows (past
// QPT G, or of entries past the item's end) read rows of the tile's first
// entry with the row offset +inf, so their P and dS are exactly 0.  A tile
// issues the same loads as a KvIssuer tile (kv_tile_loads).
template <typename T, int D, int NTH> struct GroupTiles {
  using C = Tile32<T, D>;
  static constexpr int LPT = dma_uniform_loads<NTH, C::ROW_CHUNKS>();
  struct Info {
    int e0;   // the tile's first entry
  };
  const int32_t* sent;   // the item's entries (LDS): t, or (t << sbits) | slot when packed
  int cnt, sbits, packed, G, QPT;
  const T* qg;           // Q / dO of the group (b, hkv), query 0 head 0
  const T* dg;
  const float* sp;       // statistics of the group: c for lanes < 32, delta above
  uint32_t rowbytes;     // one query's G rows in bytes
  int key, wlast, blk_end;   // this lane's key, the wave's last key, the block's end
  bool key_ok;
  int h;
  uint32_t off[LPT];     // (g D + column) * sizeof(T) of this lane's chunk of load j
  int qj[LPT];           // entry (in the tile) of that chunk's row
  int sq, sg;            // statistics row of this lane: entry and head
  bool sreal;

  __device__ __forceinline__ int entry_t(int i) const {
    if (i >= cnt) return -1;
    const int v = sent[i];
    return packed ? v >> sbits : v;
  }
  __device__ __forceinline__ int entry_s(int i) const {
    return packed && i < cnt ? sent[i] & ((1 << sbits) - 1) : 0;
  }
  __device__ __forceinline__ void prepare(int, int tid) {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int nreal = QPT * G;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int r, cc;
      row_chunk<T, D>(KvIssuer<T, D, NTH>::first_chunk(j, w) + lane, r, cc);
      const bool real = r < nreal;
      qj[j] = real ? r / G : 0;
      const int g = real ? r % G : 0;
      off[j] = (uint32_t)((g * D + cc * C::EPC) * (int)sizeof(T));
    }
    const int sr = lane & 31;
    sreal = sr < nreal;
    sq = sreal ? sr / G : 0;
    sg = sreal ? sr % G : 0;
  }
  __device__ __forceinline__ void issue(KvStage<T, D>& s, int ti, int tid) const {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int e0 = QPT * ti;
    const int t0 = __builtin_amdgcn_readfirstlane(entry_t(e0));   // a tile's first entry exists
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int t = entry_t(e0 + qj[j]);
      t = t >= 0 ? t : t0;
      const uint32_t v = (uint32_t)t * rowbytes + off[j];
      const int first = KvIssuer<T, D, NTH>::first_chunk(j, w);
      lds_dma16_sbase(qg, v, (char*)s.qr + 16 * first);
      lds_dma16_sbase(dg, v, (char*)s.dr + 16 * first);
    }
    {
      // lanes 0-31: c of row lane, lanes 32-63: delta of row lane - 32
      int t = entry_t(e0 + sq);
      const bool real = lane >= 32 || (sreal && t >= 0);
      t = t >= 0 ? t : t0;
      lds_dma4(real ? sp + (int64_t)t * G + sg : &kAbsentRow, s.c);
    }
  }
  __device__ __forceinline__ Info info(const KvStage<T, D>&, int ti) const { return Info{QPT * ti}; }
  // the rows of entries whose query the lane's key precedes; the per-element
  // test is skipped only when every key of the wave precedes every entry's query
  __device__ __forceinline__ VisBits vis(const Info& i, bool& mask) const {
    const uint32_t gmask = (1u << G) - 1u;
    uint32_t bits = 0;
    int tmin = 0x7fffffff;
    for (int q = 0; q < QPT; ++q) {
      const int t = __builtin_amdgcn_readfirstlane(entry_t(i.e0 + q));
      if (t < 0) break;   // entries past the item's end are the tile's last
      tmin = t < tmin ? t : tmin;
      if (key_ok && key <= t) bits |= gmask << (q * G);
    }
    mask = !(wlast <= tmin && wlast < blk_end);
    return VisBits{bits >> (8 * h)};
  }
};

// Walk `ntile` row tiles of each of `nhc` head chunks, kKvStages tiles deep,
// one workgroup barrier per tile, in the middle of it:
//   front(i)                     S / dP MFMAs, transposed reads, P / dS
//   wait for tile i+1, barrier   tile i+1 visible; stage i retired by every wave
//   read rows of tile i+1        LDS reads overlapping ...
//   back(i), post(i)             ... the dK / dV MFMAs
//   request tile i + kKvStages   into stage i
// Every vector-memory operation a wave issues in the loop is counted: LT
// loads per request (kv_tile_loads) and at least NSW stores per post.  The
// operations younger than tile i+1's loads are the kKvStages - 2 requests
// after it and the min(i, kKvStages - 2) posts issued since, so waiting for
// at most that many outstanding operations completes tile i + 1 while the two
// younger tiles stay in flight (operations complete in issue order; a post
// that stores more than NSW only makes the wait longer).
// The tile source (PairTiles, GroupTiles) issues a tile's loads into a stage
// (prepare(hc, tid) once per head chunk, then issue(stage, ti, tid)), names
// the tile to the consumer (info(stage, ti)) and gives this wave's mask flag
// and visibility (vis(info, mask)).  With WANT_DS, pre(dS, i) runs before the
// barrier with this lane's dS as two operand-dtype fragments (element j of
// fragment k: accumulator register 8 k + j), and post(info, hc, i) after the
// back half, so what pre stages in LDS is visible to post without a second
// barrier.
template <bool WANT_DS, int NSW, typename T, int D, int NTH, typename Tiles, typename Pre,
          typename Post>
__device__ __forceinline__ void kv_walk(KeyAcc<T, D>& acc, KvStage<T, D> (&stg)[kKvStages], Tiles& tiles, int nhc,
                                        int ntile, Pre pre, Post post, float sl2, int tid) {
  using C = Tile32<T, D>;
  constexpr int NST = kKvStages;
  constexpr int LT = kv_tile_loads<T, D, NTH>();
  static_assert(NST >= 3 && (NST - 1) * LT < 64 && (NST - 2) * (LT + NSW) < 64,
                "in-flight operations exceed the vmcnt range");
  // wave-uniform: every branch on the loop counters below is scalar
  const int total = __builtin_amdgcn_readfirstlane(ntile * nhc);
  if (total == 0) return;
  const int lane = tid & 63;
  int iti = 0, ihc = 0;   // next tile to request: tile and head chunk
  tiles.prepare(0, tid);
  auto request = [&](KvStage<T, D>& s) {
    tiles.issue(s, iti, tid);
    if (++iti == ntile) {
      iti = 0;
      if (++ihc < nhc) tiles.prepare(ihc, tid);
    }
  };
#pragma unroll
  for (int p = 0; p < NST; ++p)
    if (p < total) request(stg[p]);
  if (total >= NST)
    vm_wait<(NST - 1) * LT>();
  else
    vm_wait<0>();
  __syncthreads();
  typename KeyAcc<T, D>::Rows rows;
  KeyAcc<T, D>::read_rows(rows, stg[0], lane);
  int hc = 0, ti = 0;   // head chunk and tile of iteration `it`
  // unrolled over the stages: every stage address (and the tile parity the
  // pre / post hooks take) is a compile-time constant, so the LDS reads use
  // immediate offsets instead of per-tile address arithmetic
  static_assert(NST % 2 == 0, "the hooks' parity is the stage's");
  for (int it0 = 0; it0 < total; it0 += NST) {
#pragma unroll
    for (int p = 0; p < NST; ++p) {
      const int it = it0 + p;
      if (it >= total) break;
      const KvStage<T, D>& s = stg[p];
      const auto inf = tiles.info(s, ti);
      bool mask;
      const auto v = tiles.vis(inf, mask);
      Frag<T> ta[C::DT][2], tb[C::DT][2], pf[2], sf[2];
      if (mask)
        acc.template front<true>(s, rows, v, sl2, lane, ta, tb, pf, sf);
      else
        acc.template front<false>(s, rows, v, sl2, lane, ta, tb, pf, sf);
      if (WANT_DS) pre(sf, p);
      if (it + NST - 1 < total)
        vm_wait_steps<(NST - 2) * LT, WANT_DS ? NSW : 0, NST - 2>(it);
      else
        vm_wait<0>();
      __syncthreads();
      if (it + 1 < total) KeyAcc<T, D>::read_rows(rows, stg[(p + 1) % NST], lane);
      acc.back(ta, tb, pf, sf);
      if (WANT_DS) post(inf, hc, p);
      if (it + NST < total) request(stg[p]);
      if (++ti == ntile) {
        ti = 0;
        ++hc;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Role-split walk: two waves share a group of 32 keys.  The P-wave keeps the
// keys' K fragments and dV^T: S = Q K^T, P = exp2(S*scale*log2(e) - c), dV^T
// += dO^T P, and P goes to LDS as the 16-bit operand it is for dV (rounded
// once; half the bytes of float, which leaves room for a fourth query stage
// at two workgroups per CU).  The dS-wave keeps V and dK^T: dP =
// dO V^T before the tile's barrier, then, with the P-wave's P of the same
// tile, dS = P (dP - delta) and dK^T += Q^T dS after it.  Each wave carries
// about half of a single walker's registers, so two waves run per SIMD
// (two workgroups per CU) and one's MFMAs cover the other's dependency
// waits.  Everything a wave reads from a query stage is read before the
// barrier of that tile, so the stage is refilled after it as in kv_walk.
// ---------------------------------------------------------------------------
constexpr int kSplitStages = 4;   // query tiles in flight + 1 (74 KB: two workgroups per CU)

// P of one tile for the dS-wave, in the lane order of the P-wave's two
// 16-bit dV operand fragments: fragment f of lane L at 16-byte slot f 64 + L
// (each store / load one 16-byte access per lane, the lanes' pieces
// consecutive).  The values go as fp16, not as the bf16 operand: in the
// backward P = exp(s - lse) * sigmoid(g) <= 1, and fp16 keeps 11 significant
// bits of it where bf16 keeps 8 -- dS = P (dP - delta) is formed from them.
typedef uint32_t PTile[4 * 64 * 2];
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <typename T, int D> struct PWave {
  using C = Tile32<T, D>;
  Frag<T> kf[C::KS];
  f32x16 dv[C::DT];
  __device__ __forceinline__ void init(const T* kb, int key_safe, int h) {
#pragma unroll
    for (int s = 0; s < C::KS; ++s) kf[s].load(kb + (int64_t)key_safe * D + 16 * s + 8 * h);
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dv[dt] = zero16();
#pragma unroll
    for (int s = 0; s < C::KS; ++s) settle(kf[s]);
  }
  template <bool MASK, typename Vis>
  __device__ __forceinline__ void tile(const KvStage<T, D>& s, const Frag<T> (&qa)[C::KS], const Vis& vis,
                                       float sl2, int lane, uint32_t* pb) {
    const int h = lane >> 5;
    Frag<T> ta[C::DT][2];
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k) lds_tr_frag<T, D>(ta[dt][k], s.dr, dt, lane, k);
    f32x16 sacc = zero16();
#pragma unroll
    for (int k = 0; k < C::KS; ++k) mma32(sacc, qa[k], kf[k]);
    if constexpr (sizeof(T) == 2) {
      constexpr int NTR = 2 * C::DT * 2;
      constexpr int PER = (NTR + C::KS - 1) / C::KS;
#pragma unroll
      for (int i = 0; i < C::KS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);
      }
    }
    float P[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(sacc[r] * sl2 - s.c[acc_elem(h, r)]);
      if (MASK) p = vis(r) ? p : 0.0f;
      P[r] = p;
    }
    Frag<T> pf[2];
    pf[0].set(P);
    pf[1].set(P + 8);
    {
      static_assert(sizeof(T) == 2, "the role-split walk hands P over as 16-bit values");
      typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
      f16x8 h0, h1;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        h0[r] = (_Float16)P[r];
        h1[r] = (_Float16)P[8 + r];
      }
      *reinterpret_cast<u32x4_*>(pb + 4 * lane) = __builtin_bit_cast(u32x4_, h0);
      *reinterpret_cast<u32x4_*>(pb + 256 + 4 * lane) = __builtin_bit_cast(u32x4_, h1);
    }
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k) mma32(dv[dt], ta[dt][k], pf[k]);
  }
};

template <typename T, int D> struct SWave {
  using C = Tile32<T, D>;
  Frag<T> vf[C::KS];
  f32x16 dk[C::DT];
  __device__ __forceinline__ void init(const T* vb, int key_safe, int h) {
#pragma unroll
    for (int s = 0; s < C::KS; ++s) vf[s].load(vb + (int64_t)key_safe * D + 16 * s + 8 * h);
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dk[dt] = zero16();
#pragma unroll
    for (int s = 0; s < C::KS; ++s) settle(vf[s]);
  }
  // before the barrier: dP, and the tile's Q^T fragments and deltas
  __device__ __forceinline__ void front(const KvStage<T, D>& s, const Frag<T> (&da)[C::KS], int lane, f32x16& pacc,
                                        Frag<T> (&tb)[C::DT][2], float (&dlt)[16]) {
    const int h = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k) lds_tr_frag<T, D>(tb[dt][k], s.qr, dt, lane, k);
    pacc = zero16();
#pragma unroll
    for (int k = 0; k < C::KS; ++k) mma32(pacc, da[k], vf[k]);
    if constexpr (sizeof(T) == 2) {
      constexpr int NTR = 2 * C::DT * 2;
      constexpr int PER = (NTR + C::KS - 1) / C::KS;
#pragma unroll
      for (int i = 0; i < C::KS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) dlt[r] = s.dot[acc_elem(h, r)];
  }
  // after: dS from the P-wave's P; dK^T += Q^T dS; sf receives dS as
  // operand fragments
  __device__ __forceinline__ void back(const uint32_t* pb, const f32x16& pacc, const Frag<T> (&tb)[C::DT][2],
                                       const float (&dlt)[16], int lane, Frag<T> (&sf)[2]) {
    float dS[16];
    typedef uint32_t u32x4_ __attribute__((ext_vector_type(4)));
    f16x8 ph[2];
    ph[0] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4_*>(pb + 4 * lane));
    ph[1] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4_*>(pb + 256 + 4 * lane));
#pragma unroll
    for (int r = 0; r < 16; ++r) dS[r] = (float)ph[r >> 3][r & 7] * (pacc[r] - dlt[r]);
    sf[0].set(dS);
    sf[1].set(dS + 8);
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k) mma32(dk[dt], tb[dt][k], sf[k]);
  }
};

// The query-tile requests of a split walk: every wave of the workgroup issues
// its share of each tile (NTH threads), at the same iterations.
template <typename T, int D, int NTH, typename QSrc> struct SplitReq {
  KvIssuer<T, D, NTH> iss;
  int iti, ihc;
  const int ntile, b, hkv, tid;
  const QSide<T>& x;
  QSrc& qsrc;
  __device__ __forceinline__ SplitReq(const QSide<T>& x_, int b_, int hkv_, int ntile_, QSrc& q, int tid_)
      : iti(0), ihc(0), ntile(ntile_), b(b_), hkv(hkv_), tid(tid_), x(x_), qsrc(q) {
    iss.prepare(x, b, hkv, 0, tid);
  }
  __device__ __forceinline__ void request(KvStage<T, D>& s) {
    int tA, tB, sA, sB;
    qsrc(iti, tA, tB, sA, sB);
    iss.issue(s, x, tA, tB, sA, sB, tid);
    if (++iti == ntile) {
      iti = 0;
      if (++ihc < x.NHC) iss.prepare(x, b, hkv, ihc, tid);
    }
  }
};

// The query-tile requests of a split walk over flat rows (groups of G < 16
// heads, where two queries x 16 head slots would leave 32 - 2 G rows of a
// tile empty): the rows (t, g) of the group are numbered t G + g and tile i
// holds rows rlo + 32 i .. rlo + 32 i + 31, read from the [B, Hq, T, D]
// layout (row (t, g) at (g T + t) D from the group's first row).  Each lane
// keeps the query and head of its loads' rows and of its statistics row and
// moves them 32 rows on per request.  Rows of queries past thi (the
// workgroup's last query) read row (thi, g) with the row offset +inf, so
// their P and dS are exactly 0.  Same loads per tile as KvIssuer.
template <typename T, int D, int NTH> struct FlatReq {
  using C = Tile32<T, D>;
  static constexpr int LPT = dma_uniform_loads<NTH, C::ROW_CHUNKS>();
  const T* qg;          // Q / dO of the group: query 0, head 0
  const T* dg;
  const float* sp;      // c (lanes < 32) or delta (lanes >= 32) of the group, [G][T]
  int T_, G, thi, step_g, step_t;   // 32 rows = step_t queries + step_g heads
  int tid;
  uint32_t col[LPT];    // column byte offset of this lane's chunk of load j
  int tj[LPT], gj[LPT];  // query / head of that chunk's row in the next tile
  int ts, gs;           // query / head of this lane's statistics row in the next tile

  __device__ __forceinline__ void init(const QSide<T>& x, int b, int hkv, int rlo, int thi_, int tid_) {
    G = x.G;
    T_ = x.T_;
    thi = thi_;
    tid = tid_;
    step_t = 32 / G;
    step_g = 32 - step_t * G;
    const int64_t g0 = (int64_t)b * x.Hq + (int64_t)hkv * G;   // the group's first head
    qg = x.q + g0 * T_ * D;
    dg = x.dout + g0 * T_ * D;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    sp = (lane < 32 ? x.c : x.dot) + g0 * T_;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int r, cc;
      row_chunk<T, D>(KvIssuer<T, D, NTH>::first_chunk(j, w) + lane, r, cc);
      col[j] = (uint32_t)(cc * 16);
      tj[j] = (rlo + r) / G;
      gj[j] = rlo + r - tj[j] * G;
    }
    ts = (rlo + (lane & 31)) / G;
    gs = rlo + (lane & 31) - ts * G;
  }
  __device__ __forceinline__ void advance(int& t, int& g) const {
    g += step_g;
    t += step_t;
    if (g >= G) {
      g -= G;
      ++t;
    }
  }
  __device__ __forceinline__ void request(KvStage<T, D>& s) {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int t = tj[j] <= thi ? tj[j] : thi;
      const uint32_t v = ((uint32_t)gj[j] * (uint32_t)T_ + (uint32_t)t) * (uint32_t)(D * sizeof(T)) + col[j];
      const int first = KvIssuer<T, D, NTH>::first_chunk(j, w);
      lds_dma16_sbase(qg, v, (char*)s.qr + 16 * first);
      lds_dma16_sbase(dg, v, (char*)s.dr + 16 * first);
      advance(tj[j], gj[j]);
    }
    {
      // lanes 0-31: c of row lane, lanes 32-63: delta of row lane - 32
      const bool real = lane >= 32 || ts <= thi;
      const int t = ts <= thi ? ts : thi;
      lds_dma4(real ? sp + (int64_t)gs * T_ + t : &kAbsentRow, s.c);
      advance(ts, gs);
    }
  }
};

// One walk per role (the roles' registers are then never live at once).
// Per tile: [role work before the barrier]; wait for tile it+1; barrier;
// [role work after it]; refill the stage of tile it.  P goes through
// pbuf[it & 1].
// make_rq(): the tile requests (SplitReq, FlatReq), made in the same order
// by every wave (built inside the walk, whose registers they share); vis(stage,
// it, mask): the P-wave's visibility of tile it (VisPair, VisBits) and
// whether it needs the per-element test.
template <typename T, int D, int NTH, typename MakeReq, typename Vis>
__device__ __forceinline__ void walk_p(PWave<T, D>& pw, KvStage<T, D> (&stg)[kSplitStages], PTile* pbuf,
                                       MakeReq make_rq, int total, Vis vis, float sl2, int tid) {
  using C = Tile32<T, D>;
  constexpr int NST = kSplitStages;
  constexpr int LT = kv_tile_loads<T, D, NTH>();
  static_assert((NST - 1) * LT < 64, "in-flight operations exceed the vmcnt range");
  total = __builtin_amdgcn_readfirstlane(total);
  if (total == 0) return;
  const int lane = tid & 63, h = lane >> 5, n = lane & 31;
  auto rq = make_rq();
#pragma unroll
  for (int p = 0; p < NST; ++p)
    if (p < total) rq.request(stg[p]);
  if (total >= NST)
    vm_wait<(NST - 1) * LT>();
  else
    vm_wait<0>();
  __syncthreads();
  Frag<T> qa[C::KS];
#pragma unroll
  for (int k = 0; k < C::KS; ++k) lds_row_frag<T, D>(qa[k], stg[0].qr, n, h, k);
  // unrolled over the stages: stage and P-buffer addresses are constants
  static_assert(NST % 2 == 0, "the P buffer's parity is the stage's");
  for (int it0 = 0; it0 < total; it0 += NST) {
#pragma unroll
    for (int p = 0; p < NST; ++p) {
      const int it = it0 + p;
      if (it >= total) break;
      const KvStage<T, D>& s = stg[p];
      bool mask;
      const auto v = vis(s, it, mask);
      if (mask)
        pw.template tile<true>(s, qa, v, sl2, lane, pbuf[p & 1]);
      else
        pw.template tile<false>(s, qa, v, sl2, lane, pbuf[p & 1]);
      if (it + NST - 1 < total)
        vm_wait<(NST - 2) * LT>();
      else
        vm_wait<0>();
      __syncthreads();
      if (it + 1 < total) {
#pragma unroll
        for (int k = 0; k < C::KS; ++k) lds_row_frag<T, D>(qa[k], stg[(p + 1) % NST].qr, n, h, k);
      }
      if (it + NST < total) rq.request(stg[p]);
    }
  }
}

template <typename T, int D, int NTH, typename MakeReq>
__device__ __forceinline__ void walk_s(SWave<T, D>& sw, KvStage<T, D> (&stg)[kSplitStages], const PTile* pbuf,
                                       MakeReq make_rq, int total, int tid) {
  using C = Tile32<T, D>;
  constexpr int NST = kSplitStages;
  constexpr int LT = kv_tile_loads<T, D, NTH>();
  total = __builtin_amdgcn_readfirstlane(total);
  if (total == 0) return;
  const int lane = tid & 63, h = lane >> 5, n = lane & 31;
  auto rq = make_rq();
#pragma unroll
  for (int p = 0; p < NST; ++p)
    if (p < total) rq.request(stg[p]);
  if (total >= NST)
    vm_wait<(NST - 1) * LT>();
  else
    vm_wait<0>();
  __syncthreads();
  Frag<T> da[C::KS];
#pragma unroll
  for (int k = 0; k < C::KS; ++k) lds_row_frag<T, D>(da[k], stg[0].dr, n, h, k);
  static_assert(NST % 2 == 0, "the P buffer's parity is the stage's");
  for (int it0 = 0; it0 < total; it0 += NST) {
#pragma unroll
    for (int p = 0; p < NST; ++p) {
      const int it = it0 + p;
      if (it >= total) break;
      const KvStage<T, D>& s = stg[p];
      f32x16 pacc;
      Frag<T> tb[C::DT][2];
      float dlt[16];
      sw.front(s, da, lane, pacc, tb, dlt);
      if (it + NST - 1 < total)
        vm_wait<(NST - 2) * LT>();
      else
        vm_wait<0>();
      __syncthreads();
      Frag<T> sf[2];
      sw.back(pbuf[p & 1], pacc, tb, dlt, lane, sf);
      if (it + 1 < total) {
#pragma unroll
        for (int k = 0; k < C::KS; ++k) lds_row_frag<T, D>(da[k], stg[(p + 1) % NST].dr, n, h, k);
      }
      if (it + NST < total) rq.request(stg[p]);
    }
  }
}

template <typename T, int D>
__device__ __forceinline__ QSide<T> qside(const T* q, const T* dout, const float* c, const float* dot, int Hq,
                                          int Hkv, int T_, bool packed) {
  QSide<T> x;
  x.q = q;
  x.dout = dout;
  x.c = c;
  x.dot = dot;
  x.Hq = Hq;
  x.Hkv = Hkv;
  x.G = Hq / Hkv;
  x.NHC = (x.G + 15) / 16;
  x.T_ = T_;
  x.hs = packed ? (int64_t)D : (int64_t)T_ * D;
  x.ts = packed ? (int64_t)x.G * D : (int64_t)D;
  x.sh = packed ? 1 : T_;
  x.st = packed ? x.G : 1;
  return x;
}

// Compression dK/dV work: key block kb (keys 32 NW kb ..) is seen by queries
// t >= 32 NW kb cd + cl - 1, so query chunk ch has work for key blocks
// 0 .. cmp_active_blocks(ch) - 1; ch = -1 gives the total over all chunks.
__host__ __device__ inline int cmp_active_blocks(int T, int Lk, int chunk, int NW, int cl, int cd, int ch) {
  const int nkb = (Lk + 32 * NW - 1) / (32 * NW);
  const int nch = (T + chunk - 1) / chunk;
  if (ch < 0) {
    int tot = 0;
    for (int c = 0; c < nch; ++c) tot += cmp_active_blocks(T, Lk, chunk, NW, cl, cd, c);
    return tot;
  }
  const int last = (ch * chunk + chunk - 1 < T - 1 ? ch * chunk + chunk - 1 : T - 1) - (cl - 1);
  if (last < 0) return 0;
  const int n = last / (32 * NW * cd) + 1;
  return n < nkb ? n : nkb;
}

// xcd_remap for a grid of nlong long workgroups followed by nshort short
// ones: every XCD takes an equal, contiguous share of each, its long ones
// first (the few long ones that do not divide evenly go out first, the short
// ones that do not, last).
__device__ __forceinline__ int64_t xcd_remap_split(int64_t bid, int64_t nlong, int64_t nshort) {
  constexpr int64_t kXcd = 8;
  const int64_t lp = nlong / kXcd, sp = nshort / kXcd, lr = nlong % kXcd;
  if (bid < lr) return lp * kXcd + bid;
  bid -= lr;
  if (bid >= (lp + sp) * kXcd) return nlong + sp * kXcd + (bid - (lp + sp) * kXcd);
  const int64_t x = bid % kXcd, i = bid / kXcd;
  return i < lp ? x * lp + i : nlong + x * sp + (i - lp);
}

__host__ __device__ inline int cmp_blocks_range(int T, int Lk, int chunk, int NW, int cl, int cd, int c0, int c1) {
  int tot = 0;
  for (int c = c0; c < c1; ++c) tot += cmp_active_blocks(T, Lk, chunk, NW, cl, cd, c);
  return tot;
}

// Zeros over one key's float rows of dK and dV: the two lanes of a key
// (h = 0, 1) write one half of each row.
template <int D>
__device__ __forceinline__ void zero_rows(float* dkrow, float* dvrow, int h) {
#pragma unroll
  for (int d = h * (D / 2); d < (h + 1) * (D / 2); d += 4) {
    *reinterpret_cast<f32x4*>(dkrow + d) = zero4();
    *reinterpret_cast<f32x4*>(dvrow + d) = zero4();
  }
}

// ---------------------------------------------------------------------------
// range dK/dV: window: ceil(Lk / (32 NW)) * B*Hkv workgroups.  Compression:
// every (query chunk, key block) pair takes about as long as any other, so a
// grid of them would end in a partial round of workgroups on an otherwise idle
// GPU.  Chunks from `chs` on are split into `spl` sub-chunks and launched
// last, where their short workgroups fill that round.  Logical workgroups
// (placed on the XCDs by xcd_remap_split):
//   [0, nbh * big)  chunks < chs, per bh chunk-major
//   the rest        chunks >= chs, per bh (chunk, sub-chunk)-major
// (big / small: cmp_blocks_range over the two chunk ranges).
// ---------------------------------------------------------------------------
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_range_dkdv32(int mode, const T* __restrict__ q, const T* __restrict__ dout, const float* __restrict__ coff,
                    const float* __restrict__ dot, const T* __restrict__ k, const T* __restrict__ v,
                    float* __restrict__ dk, float* __restrict__ dv, float* __restrict__ part, int64_t part_half,
                    int Hq, int Hkv, int T_, int Lk, int chunk, int window, int cl, int cd, int nbh, int chs, int spl,
                    float sl2, float scale) {
  constexpr int NTH = 64 * NW;
  __shared__ __align__(16) KvStage<T, D> stg[kKvStages];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: its masks branch
  // 1-D grid over the (key block, query chunk) pairs that have work, per bh,
  // chunk-major: the workgroups of one chunk (which stream the same queries)
  // are consecutive, and XCD x takes a contiguous, equal share of them.  The
  // window has one chunk and uniform work per key block.
  const int nkb = (Lk + 32 * NW - 1) / (32 * NW);
  int kblk, ch, bh;
  int q0 = 0, qlen = chunk;   // compression: the workgroup's queries [q0, q0 + qlen)
  int64_t wg = blockIdx.x;    // logical workgroup (compression: its rows of the partial buffer)
  if (mode == NSA_MODE_COMPRESS) {
    const int nch = (T_ + chunk - 1) / chunk;
    const int big = cmp_blocks_range(T_, Lk, chunk, NW, cl, cd, 0, chs);
    const int per = cmp_blocks_range(T_, Lk, chunk, NW, cl, cd, chs, nch) * spl;
    wg = xcd_remap_split(blockIdx.x, (int64_t)big * nbh, (int64_t)per * nbh);
    int r, sub = 0;
    if (wg < (int64_t)big * nbh) {
      bh = (int)(wg / big);
      r = (int)(wg % big);
      for (ch = 0; ch < chs - 1; ++ch) {   // chunk ch holds the first cmp_active_blocks(.., ch) key blocks
        const int nb = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch);
        if (r < nb) break;
        r -= nb;
      }
    } else {
      const int64_t w2 = wg - (int64_t)big * nbh;
      bh = (int)(w2 / per);
      r = (int)(w2 % per);
      for (ch = chs; ch < nch - 1; ++ch) {
        const int nb = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch) * spl;
        if (r < nb) break;
        r -= nb;
      }
      const int nb = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch);
      sub = r / nb;
      r %= nb;
      qlen = (chunk + spl - 1) / spl;
    }
    kblk = r;
    q0 = ch * chunk + sub * qlen;
    if (q0 + qlen > ch * chunk + chunk) qlen = ch * chunk + chunk - q0;
  } else {
    kblk = (int)(blockIdx.x % nkb);
    ch = 0;
    bh = (int)(blockIdx.x / nkb);
  }
  const int b = bh / Hkv, hkv = bh % Hkv;
  const int k0 = kblk * 32 * NW;
  const int kw = k0 + 32 * w;
  const int key = kw + n;
  const bool key_ok = key < Lk;
  const QSide<T> x = qside<T, D>(q, dout, coff, dot, Hq, Hkv, T_, false);
  // query range of the workgroup
  int tlo, thi;
  const int klast = k0 + 32 * NW - 1 < Lk - 1 ? k0 + 32 * NW - 1 : Lk - 1;
  if (mode == NSA_MODE_WINDOW) {
    tlo = k0;
    thi = klast + window - 1;
  } else {
    tlo = k0 * cd + cl - 1;
    thi = T_ - 1;
    const int c0 = q0, c1 = q0 + qlen - 1;
    tlo = tlo > c0 ? tlo : c0;
    thi = thi < c1 ? thi : c1;
  }
  thi = thi < T_ - 1 ? thi : T_ - 1;
  // compression with a partial buffer: this workgroup's 32 NW rows of it
  // (every logical workgroup writes them, zeros when it has no query)
  float* prow = part != nullptr && mode == NSA_MODE_COMPRESS ? part + (wg * 32 * NW + (key - k0)) * D : nullptr;
  if (tlo > thi) {   // uniform over the workgroup
    if (prow != nullptr && key_ok) zero_rows<D>(prow, prow + part_half, h);
    return;
  }
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
  auto no_pre = [](const Frag<T>*, int) {};
  auto no_post = [](const auto&, int, int) {};
  auto tiles = pair_tiles<T, D, NTH>(x, b, hkv, qsrc, vis);
  kv_walk<false, 0, T, D, NTH>(acc, stg, tiles, x.NHC, ntile, no_pre, no_post, sl2, tid);
  if (key_ok) {
    if (prow != nullptr)
      acc.write(prow, prow + part_half, scale, false, h);
    else
      acc.write(dk + kvoff + (int64_t)key * D, dv + kvoff + (int64_t)key * D, scale, mode == NSA_MODE_COMPRESS, h);
  }
}

// accumulator columns of one key -> a float row (scaled; atomically when
// several workgroups add into it)
template <typename T, int D>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[Tile32<T, D>::DT], float* row, float scale,
                                           bool atomic, int h) {
  using C = Tile32<T, D>;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * dt + 8 * g4 + 4 * h;
      if (!(D % 32 == 0 || d < D)) continue;
      if (atomic) {
#pragma unroll
        for (int i = 0; i < 4; ++i) atomicAdd(row + d + i, acc[dt][4 * g4 + i] * scale);
      } else {
        *reinterpret_cast<f32x4*>(row + d) =
            (f32x4){acc[dt][4 * g4], acc[dt][4 * g4 + 1], acc[dt][4 * g4 + 2], acc[dt][4 * g4 + 3]} * scale;
      }
    }
  }
}

// k_range_dkdv32 with the role-split walk: 2 NW waves, waves < NW the
// P-waves of key groups 0 .. NW-1, the others their dS-waves.  FLAT: the
// query tiles are 32 consecutive rows t G + g of the group (FlatReq, groups
// of G < 16 heads), else two queries x 16 heads of a head chunk (SplitReq).
template <typename T, int D, int NW, bool FLAT>
__global__ __launch_bounds__(128 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_range_dkdv_split(int mode, const T* __restrict__ q, const T* __restrict__ dout, const float* __restrict__ coff,
                    const float* __restrict__ dot, const T* __restrict__ k, const T* __restrict__ v,
                    float* __restrict__ dk, float* __restrict__ dv, float* __restrict__ part, int64_t part_half,
                    int Hq, int Hkv, int T_, int Lk, int chunk, int window, int cl, int cd, int nbh, int chs, int spl,
                    float sl2, float scale) {
  constexpr int NTH = 128 * NW;
  __shared__ __align__(16) KvStage<T, D> stg[kSplitStages];
  __shared__ __align__(16) PTile pbuf[NW][2];
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool pwave = wv < NW;
  const int w = pwave ? wv : wv - NW;   // key group (wave-uniform: its masks branch)
  // 1-D grid over the (key block, query chunk) pairs that have work, per bh,
  // chunk-major: the workgroups of one chunk (which stream the same queries)
  // are consecutive, and XCD x takes a contiguous, equal share of them.  The
  // window has one chunk and uniform work per key block.
  const int nkb = (Lk + 32 * NW - 1) / (32 * NW);
  int kblk, ch, bh;
  int q0 = 0, qlen = chunk;   // compression: the workgroup's queries [q0, q0 + qlen)
  int64_t wg = blockIdx.x;    // logical workgroup (compression: its rows of the partial buffer)
  if (mode == NSA_MODE_COMPRESS) {
    const int nch = (T_ + chunk - 1) / chunk;
    const int big = cmp_blocks_range(T_, Lk, chunk, NW, cl, cd, 0, chs);
    const int per = cmp_blocks_range(T_, Lk, chunk, NW, cl, cd, chs, nch) * spl;
    wg = xcd_remap_split(blockIdx.x, (int64_t)big * nbh, (int64_t)per * nbh);
    int r, sub = 0;
    if (wg < (int64_t)big * nbh) {
      bh = (int)(wg / big);
      r = (int)(wg % big);
      for (ch = 0; ch < chs - 1; ++ch) {   // chunk ch holds the first cmp_active_blocks(.., ch) key blocks
        const int nb = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch);
        if (r < nb) break;
        r -= nb;
      }
    } else {
      const int64_t w2 = wg - (int64_t)big * nbh;
      bh = (int)(w2 / per);
      r = (int)(w2 % per);
      for (ch = chs; ch < nch - 1; ++ch) {
        const int nb = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch) * spl;
        if (r < nb) break;
        r -= nb;
      }
      const int nb = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch);
      sub = r / nb;
      r %= nb;
      qlen = (chunk + spl - 1) / spl;
    }
    kblk = r;
    q0 = ch * chunk + sub * qlen;
    if (q0 + qlen > ch * chunk + chunk) qlen = ch * chunk + chunk - q0;
  } else {
    kblk = (int)(blockIdx.x % nkb);
    ch = 0;
    bh = (int)(blockIdx.x / nkb);
  }
  const int b = bh / Hkv, hkv = bh % Hkv;
  const int k0 = kblk * 32 * NW;
  const int kw = k0 + 32 * w;
  const int key = kw + n;
  const bool key_ok = key < Lk;
  const QSide<T> x = qside<T, D>(q, dout, coff, dot, Hq, Hkv, T_, false);
  // query range of the workgroup
  int tlo, thi;
  const int klast = k0 + 32 * NW - 1 < Lk - 1 ? k0 + 32 * NW - 1 : Lk - 1;
  if (mode == NSA_MODE_WINDOW) {
    tlo = k0;
    thi = klast + window - 1;
  } else {
    tlo = k0 * cd + cl - 1;
    thi = T_ - 1;
    const int c0 = q0, c1 = q0 + qlen - 1;
    tlo = tlo > c0 ? tlo : c0;
    thi = thi < c1 ? thi : c1;
  }
  thi = thi < T_ - 1 ? thi : T_ - 1;
  // compression with a partial buffer: this workgroup's 32 NW rows of it
  // (every logical workgroup writes them, zeros when it has no query)
  float* prow = part != nullptr && mode == NSA_MODE_COMPRESS ? part + (wg * 32 * NW + (key - k0)) * D : nullptr;
  if (tlo > thi) {   // uniform over the workgroup
    if (prow != nullptr && key_ok) zero_rows<D>(prow, prow + part_half, h);
    return;
  }
  const int64_t kvoff = (int64_t)bh * Lk * D;
  const int wlast = kw + 31;   // last key of the group (may pass Lk: those columns are never stored)
  const int key_safe = key_ok ? key : Lk - 1;
  const bool atomic = mode == NSA_MODE_COMPRESS && prow == nullptr;
  // the two roles' walks over the workgroup's query tiles
  auto run = [&](auto make_rq, int total, auto vis) {
    if (pwave) {
      PWave<T, D> pw;
      pw.init(k + kvoff, key_safe, h);
      walk_p<T, D, NTH>(pw, stg, pbuf[w], make_rq, total, vis, sl2, tid);
      if (key_ok) store_rows<T, D>(pw.dv, prow ? prow + part_half : dv + kvoff + (int64_t)key * D, 1.0f, atomic, h);
    } else {
      SWave<T, D> sw;
      sw.init(v + kvoff, key_safe, h);
      walk_s<T, D, NTH>(sw, stg, pbuf[w], make_rq, total, tid);
      if (key_ok) store_rows<T, D>(sw.dk, prow ? prow : dk + kvoff + (int64_t)key * D, scale, atomic, h);
    }
  };
  if constexpr (FLAT) {
    // rows tlo G .. thi G + G - 1 of the group; the rows that see a key are
    // one run (flat_rows_seeing)
    const int G = x.G;
    const int rlo = tlo * G, rhi = thi * G + G - 1;
    auto make_rq = [&]() {
      FlatReq<T, D, NTH> rq;
      rq.init(x, b, hkv, rlo, thi, tid);
      return rq;
    };
    const int wmode = mode == NSA_MODE_WINDOW ? window : 0;
    auto vis = [&](const KvStage<T, D>&, int it, bool& mask) {
      const int R0 = rlo + 32 * it;
      mask = flat_tile_needs_mask(kw, R0, rhi, G, wmode, cl, cd);
      const uint32_t bits = key_ok ? flat_rows_seeing(key, R0, G, wmode, cl, cd) : 0u;
      return VisBits{bits >> (8 * h)};
    };
    run(make_rq, (rhi - rlo) / 32 + 1, vis);
  } else {
    auto qsrc = [&](int i, int& tA, int& tB, int& sA, int& sB) {
      tA = tlo + 2 * i;
      tB = tA + 1 <= thi ? tA + 1 : -1;
      sA = sB = 0;
    };
    auto vis = [&](const KvStage<T, D>& s, int, bool& mask) {
      const int tA = __builtin_amdgcn_readfirstlane(s.meta[0]), tB = __builtin_amdgcn_readfirstlane(s.meta[1]);
      const int tb = tB >= 0 ? tB : tA;
      VisPair v;
      if (mode == NSA_MODE_WINDOW) {
        mask = !(tA >= wlast && tb - window < kw);
        v.a = key <= tA && key > tA - window;
        v.b = key <= tb && key > tb - window;
      } else {
        mask = !(wlast * cd + cl - 1 <= tA);
        v.a = key * cd + cl - 1 <= tA;
        v.b = key * cd + cl - 1 <= tb;
      }
      return v;
    };
    const int ntile = (thi - tlo) / 2 + 1;
    auto make_rq = [&]() { return SplitReq<T, D, NTH, decltype(qsrc)>(x, b, hkv, ntile, qsrc, tid); };
    run(make_rq, ntile * x.NHC, vis);
  }
}

// x: 16-byte aligned; 16-byte stores for the first n & ~3 elements, the rest one by one
__global__ __launch_bounds__(256) void k_fill_zero(float* __restrict__ x, int64_t n) {
  const int64_t n4 = n >> 2;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n4; e += (int64_t)gridDim.x * 256)
    reinterpret_cast<f32x4*>(x)[e] = zero4();
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) x[(n4 << 2) + threadIdx.x] = 0.0f;
}

// Zero-fill with a kernel (safe inside captured graphs, unlike a memset node).
// x is the start of a float allocation of this library's callers (16-byte aligned).
static inline int zero_f32(float* x, int64_t n, hipStream_t s) {
  if (n <= 0) return NSA_OK;
  if (((uintptr_t)x & 15) != 0) return NSA_ERR_ARG;
  int64_t g = ((n >> 2) + 255) / 256;
  if (g > 16384) g = 16384;
  if (g < 1) g = 1;
  k_fill_zero<<<(unsigned)g, 256, 0, s>>>(x, n);
  return hipGetLastError() == hipSuccess ? NSA_OK : NSA_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// selection dK/dV over CSR work items (nsa_items.h)
// ---------------------------------------------------------------------------
// Persistent grid over the work items (next_item); two waves own 64 keys of the item's
// block at a time (blocks longer than 64 keys take several passes).  With
// dq_part, the tile's dS^T (both waves, 64 keys x 32 rows) is staged in LDS
// before the tile's barrier (double-buffered by tile parity) and dQ^T =
// K^T dS^T is formed after it for the pass's 64 keys -- each wave covering
// half of D -- and written, scaled, to the (query, slot, pass) partial that
// k_sel_dq_reduce sums.  dS enters dK^T once, as a 16-bit operand: with the
// row dots formed from fp16 branch outputs and partials, a second product
// with its rounding remainder no longer paid for its MFMAs.
// GP: groups of G <= 10 heads take floor(32 / G) entries per row tile
// (GroupTiles), the others two queries x 16 heads per head chunk (PairTiles).
template <typename T, int D, bool GP>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_sel_dkdv32(const T* __restrict__ q, const T* __restrict__ dout, const float* __restrict__ coff,
                  const float* __restrict__ dot, const T* __restrict__ k, const T* __restrict__ v,
                  const T* __restrict__ kt, const int32_t* __restrict__ q_of_block, const int4* __restrict__ items,
                  int32_t* __restrict__ n_items, float* __restrict__ dk, float* __restrict__ dv,
                  float* __restrict__ part, int64_t part_half, T* __restrict__ dq_part, int Hq, int Hkv, int T_,
                  int S, int packed, int n_blk, int L, int Lp, float sl2, float scale) {
  constexpr int NW = 2, NTH = 64 * NW;
  using C = Tile32<T, D>;
  constexpr int DT = C::DT, DTW = (DT + 1) / 2;          // dQ^T d-tiles per wave
  using CS = Tile32<T, 32>;                              // dS^T tiles: [keys][32 rows]
  __shared__ __align__(16) KvStage<T, D> stg[kKvStages];
  __shared__ __align__(16) T sdT[2][64 * 32];            // double-buffered by tile parity
  __shared__ int32_t sent[kSelItemMax];                  // the item's CSR entries
  // dQ^T partial stores per post and wave (a lower bound over the waves)
  constexpr int NSW = D >= 64 ? DTW * 2 : 0;
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, n = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const QSide<T> x = qside<T, D>(q, dout, coff, dot, Hq, Hkv, T_, true);   // packed Q / dO / statistics
  const int G = x.G;
  const int ni = *n_items;
  const int npass = sel_passes(L);
  const int NS = S * npass;
  const int sbits = sel_slot_bits(S);
  __shared__ int next_slot;
  for (int it = blockIdx.x; it < ni * npass; it = next_item(n_items + 1, &next_slot)) {
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
    const int beg = item.y, cnt = item.z - item.y;
    // the item's entries go to LDS once: a global load per tile would be
    // waited for with every tile load in flight
    for (int i = tid; i < cnt; i += NTH) sent[i] = q_of_block[beg + i];
    KeyAcc<T, D> acc;
    acc.init(k + kvoff, v + kvoff, key_ok ? key : j * L, h);
    // K^T fragments of the pass's 64 keys for this wave's dQ^T d-tiles, rows
    // in perm32 order (each lane's outputs are then 8 consecutive d: 16-byte
    // stores)
    Frag<T> ktf[DTW][4];
    if (dq_part != nullptr) {
      const T* ktb = kt + (int64_t)bh * D * Lp;
#pragma unroll
      for (int i = 0; i < DTW; ++i)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int d = 32 * (w * DTW + i) + perm32(n);
          int c0 = kpass + 16 * kk + 8 * h;
          c0 = c0 < Lp - 8 ? c0 : Lp - 8;
          if (w * DTW + i < DT && (D % 32 == 0 || d < D))
            ktf[i][kk].load(ktb + (int64_t)d * Lp + c0);
          else
            ktf[i][kk].zero();
        }
    }
    if (dq_part != nullptr) {
#pragma unroll
      for (int i = 0; i < DTW; ++i)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) settle(ktf[i][kk]);
    }
    __syncthreads();   // sent visible to every wave
    // dS^T (this wave's 32 keys x the tile's 32 rows) -> LDS, two 16-byte
    // pieces per lane: row 32 w + n of sdT, elements 8 h .. and 16 + 8 h ..
    auto pre = [&](const Frag<T>* ds, int i) {
      T* tile = sdT[i & 1] + (32 * w) * 32;
      const int r = n;   // row of this wave's 32-key sub-tile
#pragma unroll
      for (int kf = 0; kf < 2; ++kf) {
        if constexpr (sizeof(T) == 2) {
          const int c = (16 * kf + 8 * h) / CS::EPC;
          *reinterpret_cast<bf16x8*>(tile + r * 32 + (c ^ CS::rkey(r)) * CS::EPC) = ds[kf].v;
        } else {
          const int c = (16 * kf + 8 * h) / CS::EPC;
          *reinterpret_cast<f32x4*>(tile + r * 32 + (c ^ CS::rkey(r)) * CS::EPC) = ds[kf].lo;
          *reinterpret_cast<f32x4*>(tile + r * 32 + ((c + 1) ^ CS::rkey(r)) * CS::EPC) = ds[kf].hi;
        }
      }
    };
    // dQ^T = K^T dS^T over the pass's 64 keys, this wave's d-tiles, from the
    // dS^T that pre staged for tile parity i; lane (h, n) holds row n
    auto dq_tile = [&](f32x16 (&dq)[DTW], int i) {
#pragma unroll
      for (int d = 0; d < DTW; ++d) dq[d] = zero16();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        Frag<T> bf;
        lds_tr_frag<T, 32>(bf, sdT[i & 1] + (kk >> 1) * 32 * 32, 0, lane, kk & 1);
#pragma unroll
        for (int d = 0; d < DTW; ++d) mma32(dq[d], ktf[d][kk], bf);
      }
    };
    // ... written scaled to head g of the (query t, partial slot) partial
    auto dq_store = [&](const f32x16 (&dq)[DTW], int t, int slot, int g) {
      T* drow = dq_part + ((((int64_t)bh * T_ + t) * NS + slot) * G + g) * D;
      // register r of lane half h holds d = 32 (w DTW + d) + acc_elem(h, r)
#pragma unroll
      for (int d = 0; d < DTW; ++d) {
        if (w * DTW + d >= DT) continue;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int dd = 32 * (w * DTW + d) + 16 * hf + 8 * h;
          float y[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) y[i] = dq[d][8 * hf + i] * scale;
          if (D % 32 == 0 || dd < D) store8(drow + dd, y);
        }
      }
    };
    if constexpr (GP) {
      const int QPT = 32 / G;
      const int64_t grow = (int64_t)bh * G * T_;   // the group's first packed row
      GroupTiles<T, D, NTH> tiles;
      tiles.sent = sent;
      tiles.cnt = cnt;
      tiles.sbits = sbits;
      tiles.packed = packed;
      tiles.G = G;
      tiles.QPT = QPT;
      tiles.qg = x.q + grow * D;
      tiles.dg = x.dout + grow * D;
      tiles.sp = (lane < 32 ? x.c : x.dot) + grow;
      tiles.rowbytes = (uint32_t)(G * D * (int)sizeof(T));
      tiles.key = key;
      tiles.wlast = wlast;
      tiles.blk_end = blk_end;
      tiles.key_ok = key_ok;
      tiles.h = h;
      const int ntile = (cnt + QPT - 1) / QPT;
      const int pq = n / G, pg = n % G;   // this lane's dQ row: entry and head
      const bool preal = n < QPT * G;
      auto post = [&](const typename GroupTiles<T, D, NTH>::Info& inf, int, int i) {
        f32x16 dq[DTW];
        dq_tile(dq, i);
        const int e = inf.e0 + pq;
        const int t = tiles.entry_t(e);
        if (preal && t >= 0) dq_store(dq, t, tiles.entry_s(e) * npass + pass, pg);
      };
      if (dq_part != nullptr)
        kv_walk<true, NSW, T, D, NTH>(acc, stg, tiles, 1, ntile, pre, post, sl2, tid);
      else
        kv_walk<false, 0, T, D, NTH>(acc, stg, tiles, 1, ntile, pre, post, sl2, tid);
    } else {
      const int ntile = (cnt + 1) / 2;
      auto decode = [&](int i, int& t, int& s) {
        if (i < cnt) {
          const int val = sent[i];
          t = packed ? val >> sbits : val;
          s = packed ? val & ((1 << sbits) - 1) : 0;
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
        // the per-element test is skipped only when every key of the wave
        // precedes both queries (the earlier of the two: the entries' order is
        // not relied on)
        mask = !(wlast <= (tA < tb ? tA : tb) && wlast < blk_end);
        visA = key_ok && key <= tA;
        visB = key_ok && key <= tb;
      };
      auto post = [&](const auto& inf, int hc, int i) {
        f32x16 dq[DTW];
        dq_tile(dq, i);
        const int t = n < 16 ? inf.tA : inf.tB;
        const int g = hc * 16 + (n & 15);
        if (t >= 0 && g < G) dq_store(dq, t, (n < 16 ? inf.sA : inf.sB) * npass + pass, g);
      };
      auto tiles = pair_tiles<T, D, NTH>(x, b, hkv, qsrc, vis);
      if (dq_part != nullptr)
        kv_walk<true, NSW, T, D, NTH>(acc, stg, tiles, x.NHC, ntile, pre, post, sl2, tid);
      else
        kv_walk<false, 0, T, D, NTH>(acc, stg, tiles, x.NHC, ntile, pre, post, sl2, tid);
    }
    if (key_ok) {
      if (part != nullptr) {
        // this item's rows of the partial buffer (k_sel_dkdv_reduce sums them
        // in item order)
        float* pr = part + ((int64_t)it * kSelPass + (key - kpass)) * D;
        acc.write(pr, pr + part_half, scale, false, h);
      } else {
        acc.write(dk + kvoff + (int64_t)key * D, dv + kvoff + (int64_t)key * D, scale, true, h);
      }
    }
    __syncthreads();   // the next item's first tiles reuse stages 0 .. and sent
  }
}

// dK / dV of every key of the selection blocks from the work items'
// partials: one thread per 4 floats of a key row, each summed over the
// block's items in item order (the items of a block are consecutive and
// ascend in query order), so the result does not depend on which workgroup
// finished first.  A block no query selected gets zeros.
template <int D>
__global__ __launch_bounds__(256) void k_sel_dkdv_reduce(const float* __restrict__ part, int64_t part_half,
                                                         const int32_t* __restrict__ first, float* __restrict__ dk,
                                                         float* __restrict__ dv, int T_, int n_blk, int L, int npass,
                                                         int64_t total) {
  constexpr int V4 = D / 4;   // float4 per key row
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (f >= total) return;
  const int c = (int)(f % V4);
  const int kk = (int)((f / V4) % kSelPass);
  const int64_t ep = f / ((int64_t)V4 * kSelPass);   // (block, pass)
  const int e = (int)(ep / npass), pass = (int)(ep % npass);   // e = bh * n_blk + j
  const int bh = e / n_blk, j = e % n_blk;
  const int key = j * L + kSelPass * pass + kk;
  const int kend = j * L + L < T_ ? j * L + L : T_;
  if (kSelPass * pass + kk >= L || key >= kend) return;
  const int i0 = first[e], i1 = first[e + 1];
  f32x4 a = zero4(), b = zero4();
  for (int i = i0; i < i1; ++i) {
    const int64_t row = ((int64_t)i * npass + pass) * kSelPass + kk;
    a += reinterpret_cast<const f32x4*>(part + row * D)[c];
    b += reinterpret_cast<const f32x4*>(part + part_half + row * D)[c];
  }
  const int64_t orow = ((int64_t)bh * T_ + key) * D;
  reinterpret_cast<f32x4*>(dk + orow)[c] = a;
  reinterpret_cast<f32x4*>(dv + orow)[c] = b;
}

// dK / dV of the pooled keys from the compression workgroups' partial rows:
// one thread per 4 floats of a key row, summed over the key block's chunks in
// chunk (then sub-chunk) order -- the logical workgroup numbering of
// k_range_dkdv32 / k_range_dkdv_split -- so the result does not depend on
// which workgroup finished first.
template <int D, int NW>
__global__ __launch_bounds__(256) void k_cmp_dkdv_reduce(const float* __restrict__ part, int64_t part_half,
                                                         float* __restrict__ dk, float* __restrict__ dv, int T_,
                                                         int Lk, int chunk, int cl, int cd, int nbh, int chs,
                                                         int spl) {
  constexpr int KB = 32 * NW;
  constexpr int V4 = D / 4;   // float4 per key row
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (f >= (int64_t)nbh * Lk * V4) return;
  const int c = (int)(f % V4);
  const int key = (int)((f / V4) % Lk);
  const int bh = (int)(f / ((int64_t)V4 * Lk));
  const int kblk = key / KB, kk = key % KB;
  const int nch = (T_ + chunk - 1) / chunk;
  const int big = cmp_blocks_range(T_, Lk, chunk, NW, cl, cd, 0, chs);
  const int per = cmp_blocks_range(T_, Lk, chunk, NW, cl, cd, chs, nch) * spl;
  f32x4 a = zero4(), b = zero4();
  auto add = [&](int64_t wgi) {
    const int64_t row = wgi * KB + kk;
    a += reinterpret_cast<const f32x4*>(part + row * D)[c];
    b += reinterpret_cast<const f32x4*>(part + part_half + row * D)[c];
  };
  int64_t base = (int64_t)bh * big;   // chunks < chs: per bh, chunk-major
  for (int ch = 0; ch < chs; ++ch) {
    const int na = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch);
    if (kblk < na) add(base + kblk);
    base += na;
  }
  base = (int64_t)big * nbh + (int64_t)bh * per;   // the split chunks: (chunk, sub-chunk)-major
  for (int ch = chs; ch < nch; ++ch) {
    const int na = cmp_active_blocks(T_, Lk, chunk, NW, cl, cd, ch);
    if (kblk < na)
      for (int sub = 0; sub < spl; ++sub) add(base + (int64_t)sub * na + kblk);
    base += (int64_t)na * spl;
  }
  const int64_t orow = ((int64_t)bh * Lk + key) * D;
  reinterpret_cast<f32x4*>(dk + orow)[c] = a;
  reinterpret_cast<f32x4*>(dv + orow)[c] = b;
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

static constexpr int kCmpChunk = 2048;   // queries per compression dK/dV work item
static constexpr int kCmpSplit = 4;      // sub-chunks of the chunks that end the grid

// Device of a stream (the null stream: the current device), or -1.
static int stream_device(hipStream_t s) {
  hipDevice_t dev = -1;
  if (hipStreamGetDevice(s, &dev) != hipSuccess) return -1;
  return (int)dev;
}

// Compute units of the stream's device, cached per device.  The cache is
// written with relaxed atomics: two threads that race on a first lookup store
// the same value.
static int device_cu_count(hipStream_t s) {
  static std::atomic<int> cache[64];
  const int dev = stream_device(s);
  if (dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}


// Compression dK/dV grid: logical workgroups over (key block, query chunk),
// the chunks from *chs on split into *spl sub-chunks while their workgroups fit
// in one round of the resident workgroups (two per CU of the stream's device).
static int64_t cmp_grid(int T, int Lk, int cl, int cd, int nbh, hipStream_t s, int* chs_out, int* spl_out) {
  constexpr int NW = 2;
  const int nch = (T + kCmpChunk - 1) / kCmpChunk;
  const int64_t slots = 2 * (int64_t)device_cu_count(s);
  int64_t tail = 0;
  int chs = nch;
  while (chs > 0) {
    const int64_t add = (int64_t)cmp_active_blocks(T, Lk, kCmpChunk, NW, cl, cd, chs - 1) * nbh;
    if (tail + add > slots) break;
    tail += add;
    --chs;
  }
  const int spl = chs < nch ? kCmpSplit : 1;
  *chs_out = chs;
  *spl_out = spl;
  return ((int64_t)cmp_blocks_range(T, Lk, kCmpChunk, NW, cl, cd, 0, chs) +
          (int64_t)cmp_blocks_range(T, Lk, kCmpChunk, NW, cl, cd, chs, nch) * spl) * nbh;
}

extern "C" {

size_t nsa_range_dkdv_partial_bytes(int mode, int B, int Hkv, int T, int Lk, int D, int cmp_block, int cmp_stride,
                                    void* stream) {
  if (mode != NSA_MODE_COMPRESS || B <= 0 || Hkv <= 0 || T <= 0 || Lk <= 0 || D <= 0 || cmp_block < 1 ||
      cmp_stride < 1)
    return 0;
  int chs = 0, spl = 1;
  const int64_t grid = cmp_grid(T, Lk, cmp_block, cmp_stride, B * Hkv, (hipStream_t)stream, &chs, &spl);
  return (size_t)grid * 64 * (size_t)D * 2 * sizeof(float);
}

int nsa_range_dkdv(int mode, const void* q, const void* k, const void* v, const void* dout, const float* coff,
                   const float* dot, float* dk, float* dv, float* dkdv_part, size_t part_bytes, int B, int Hq, int Hkv,
                   int T, int Lk, int D, int window, int cmp_block, int cmp_stride, int dtype, void* stream) {
  NSA_CHECK(mode == NSA_MODE_WINDOW || mode == NSA_MODE_COMPRESS, NSA_ERR_ARG);
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && Lk >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(mode == NSA_MODE_COMPRESS || (window >= 1 && Lk == T), NSA_ERR_SHAPE);
  NSA_CHECK(mode == NSA_MODE_WINDOW || (cmp_block >= 1 && cmp_stride >= 1), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  // the tile loads address a group's Q / dO rows with 32-bit byte offsets
  NSA_CHECK((int64_t)(Hq / Hkv) * T * D * (dtype == NSA_BF16 ? 2 : 4) < (1ll << 32), NSA_ERR_SHAPE);
  hipStream_t s = (hipStream_t)stream;
  const int64_t nel = (int64_t)B * Hkv * Lk * D;
  // 64 keys (NW = 2 groups of 32) per workgroup, two workgroups per CU: 2 waves
  // (one per group, float) or 4 (P- and dS-wave per group, bf16).  Measured
  // faster than 128 keys sharing each streamed query tile, for both modes and
  // both walks; the role-split walk takes config 3's window / compression
  // dK/dV from 2.03 / 3.89 ms to 1.72 / 3.18 ms, and unrolled over its
  // stages to 1.61 / 3.03 ms.
  constexpr int NW = 2;
  const int nbh = B * Hkv;
  int chs = 0, spl = 1;
  int64_t grid = 0;
  if (T > 0 && Lk > 0)
    grid = mode == NSA_MODE_COMPRESS ? cmp_grid(T, Lk, cmp_block, cmp_stride, nbh, s, &chs, &spl)
                                     : (int64_t)((Lk + 32 * NW - 1) / (32 * NW)) * nbh;
  // compression partials: the workgroups write their rows, k_cmp_dkdv_reduce
  // sums them in a fixed order and writes every key
  const bool partial = mode == NSA_MODE_COMPRESS && dkdv_part != nullptr && grid > 0;
  NSA_CHECK(!partial || part_bytes >= (size_t)grid * 64 * D * 2 * sizeof(float), NSA_ERR_WORKSPACE);
  if ((mode == NSA_MODE_COMPRESS && !partial) || T == 0) {
    int rc = zero_f32(dk, nel, s);
    if (rc == NSA_OK) rc = zero_f32(dv, nel, s);
    if (rc != NSA_OK) return rc;
  }
  if (grid == 0) return NSA_OK;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  float* part = partial ? dkdv_part : nullptr;
  const int64_t part_half = grid * 32 * NW * D;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16) {
      // groups of G < 16 heads: query tiles of 32 consecutive (query, head) rows
      auto kern = Hq / Hkv < 16 ? k_range_dkdv_split<bf16, DD, NW, true> : k_range_dkdv_split<bf16, DD, NW, false>;
      kern<<<(unsigned)grid, 128 * NW, 0, s>>>(mode, (const bf16*)q, (const bf16*)dout, coff, dot, (const bf16*)k,
                                               (const bf16*)v, dk, dv, part, part_half, Hq, Hkv, T, Lk, kCmpChunk,
                                               window, cmp_block, cmp_stride, nbh, chs, spl, sl2, scale);
    } else
      k_range_dkdv32<float, DD, NW><<<(unsigned)grid, 64 * NW, 0, s>>>(
          mode, (const float*)q, (const float*)dout, coff, dot, (const float*)k, (const float*)v, dk, dv, part,
          part_half, Hq, Hkv, T, Lk, kCmpChunk, window, cmp_block, cmp_stride, nbh, chs, spl, sl2, scale);
    if (partial) {
      if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
      const int64_t total = (int64_t)nbh * Lk * (DD / 4);
      k_cmp_dkdv_reduce<DD, NW><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
          part, part_half, dk, dv, T, Lk, kCmpChunk, cmp_block, cmp_stride, nbh, chs, spl);
    }
  });
  return nsa_launch_status();
}

size_t nsa_sel_dkdv_workspace(int B, int Hkv, int T, int S, int block_size, int chunk) {
  if (B <= 0 || Hkv <= 0 || T < 0 || S < 0 || block_size <= 0 || chunk <= 0) return 0;
  const size_t nb = (size_t)B * Hkv * sel_csr_blocks(T, block_size);
  return sel_items_cap(B, Hkv, T, S, block_size, chunk) * sizeof(int4) + 256 + (nb + 1) * sizeof(int32_t);
}

size_t nsa_sel_dkdv_partial_bytes(int B, int Hkv, int T, int S, int D, int block_size, int chunk) {
  if (B <= 0 || Hkv <= 0 || T < 0 || S < 0 || D <= 0 || block_size <= 0 || chunk <= 0) return 0;
  return sel_items_cap(B, Hkv, T, S, block_size, chunk) * sel_passes(block_size) * kSelPass * (size_t)D * 2 *
         sizeof(float);
}

int nsa_sel_dkdv(const void* q, const void* k, const void* v, const void* kt, const void* dout, const float* coff,
                 const float* dot, const int32_t* q_of_block, int packed, const int32_t* block_offsets, const int32_t* pair_count,
                 float* dk, float* dv, float* dkdv_part, size_t part_bytes, void* dq_part, void* workspace,
                 size_t workspace_bytes, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                 int dtype, void* stream) {
  (void)pair_count;
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && S >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 16 || D == 32 || D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(block_size >= 16 && block_size % 16 == 0 && chunk >= 2 && chunk <= kSelItemMax, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(workspace_bytes >= nsa_sel_dkdv_workspace(B, Hkv, T, S, block_size, chunk), NSA_ERR_WORKSPACE);
  NSA_CHECK(dkdv_part == nullptr || part_bytes >= nsa_sel_dkdv_partial_bytes(B, Hkv, T, S, D, block_size, chunk),
            NSA_ERR_WORKSPACE);
  NSA_CHECK(dq_part == nullptr || (packed && kt != nullptr), NSA_ERR_ARG);
  NSA_CHECK(!packed || ((int64_t)T << sel_slot_bits(S)) < (1ll << 31), NSA_ERR_SHAPE);
  // the tile loads address a group's Q / dO rows with 32-bit byte offsets
  NSA_CHECK((int64_t)(Hq / Hkv) * T * D * (dtype == NSA_BF16 ? 2 : 4) < (1ll << 32), NSA_ERR_SHAPE);
  hipStream_t s = (hipStream_t)stream;
  const int64_t nel = (int64_t)B * Hkv * T * D;
  const int n_blk = sel_csr_blocks(T, block_size);
  const bool empty = T == 0 || S == 0 || n_blk == 0;
  if (dkdv_part == nullptr || empty) {
    // atomics add into zeroed outputs (the partial reduce writes every key)
    int rc = zero_f32(dk, nel, s);
    if (rc == NSA_OK) rc = zero_f32(dv, nel, s);
    if (rc != NSA_OK) return rc;
  }
  if (empty) return NSA_OK;
  const size_t cap = sel_items_cap(B, Hkv, T, S, block_size, chunk);
  int4* items = (int4*)workspace;
  int32_t* n_items = (int32_t*)((char*)workspace + cap * sizeof(int4));
  int32_t* first = (int32_t*)((char*)workspace + cap * sizeof(int4) + 256);
  const int nb = B * Hkv * n_blk;
  k_sel_items<<<1, 1024, 0, s>>>(block_offsets, nb, n_blk, chunk, items, n_items, first);
  if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
  const int64_t part_half = (int64_t)cap * sel_passes(block_size) * kSelPass * D;
  // one workgroup per resident slot (two per CU); next_item hands out the rest
  const size_t slots = 2 * (size_t)device_cu_count(s);
  const size_t grid_cap = cap * sel_passes(block_size) < slots ? cap * sel_passes(block_size) : slots;
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  const int Lp = padded_len(T);
  // groups of up to 10 heads pack floor(32 / G) >= 3 entries into a row tile
  const bool gp = Hq / Hkv <= kGroupPackMaxG;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16) {
      auto kern = gp ? k_sel_dkdv32<bf16, DD, true> : k_sel_dkdv32<bf16, DD, false>;
      kern<<<(unsigned)grid_cap, 128, 0, s>>>(
          (const bf16*)q, (const bf16*)dout, coff, dot, (const bf16*)k, (const bf16*)v, (const bf16*)kt, q_of_block,
          items, n_items, dk, dv, dkdv_part, part_half, (bf16*)dq_part, Hq, Hkv, T, S, packed, n_blk, block_size,
          Lp, sl2, scale);
    } else {
      auto kern = gp ? k_sel_dkdv32<float, DD, true> : k_sel_dkdv32<float, DD, false>;
      kern<<<(unsigned)grid_cap, 128, 0, s>>>(
          (const float*)q, (const float*)dout, coff, dot, (const float*)k, (const float*)v, (const float*)kt,
          q_of_block, items, n_items, dk, dv, dkdv_part, part_half, (float*)dq_part, Hq, Hkv, T, S, packed, n_blk,
          block_size, Lp, sl2, scale);
    }
    if (dkdv_part != nullptr) {
      if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
      const int npass = sel_passes(block_size);
      const int64_t total = (int64_t)nb * npass * kSelPass * (DD / 4);
      k_sel_dkdv_reduce<DD><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(dkdv_part, part_half, first, dk, dv, T,
                                                                              n_blk, block_size, npass, total);
    }
  });
  return nsa_launch_status();
}

}  // extern "C"

// ---------------------------------------------------------------------------
// nsa_sel_dkdv without a caller workspace
// ---------------------------------------------------------------------------
// The work-item list and the item counters of nsa_sel_dkdv live in this
// file-scope device array instead of the caller's workspace.  Each GPU holds
// its own copy until the process ends.  Host code never passes the array's
// name to a kernel or a copy (on the host it is a stand-in, not a device
// address): the address comes from hipGetSymbolAddress, looked up once per
// device with that device current, and kept per device.
constexpr size_t kSelScratchBytes = NSA_SEL_NOALLOC_SCRATCH_BYTES;   // 65520 work items + the counters
static __device__ __align__(256) char scratch[kSelScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// Device address of `scratch` on the device of stream `s`, looked up on first
// use with that device current (the caller's current device is restored).
int scratch_on_stream_device(hipStream_t s, void** out) {
  const int dev = stream_device(s);
  if (dev < 0 || dev >= kMaxDevices) return NSA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return NSA_ERR_LAUNCH;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return NSA_ERR_LAUNCH;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return NSA_ERR_LAUNCH;
    if (e != hipSuccess || p == nullptr) return NSA_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NSA_OK;
}
}  // namespace

extern "C" {

int nsa_sel_dkdv_noalloc(const void* q, const void* k, const void* v, const void* kt, const void* dout,
                         const float* coff, const float* dot, const int32_t* q_of_block, int packed,
                         const int32_t* block_offsets, const int32_t* pair_count, float* dk, float* dv,
                         void* dq_part, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                         int dtype, void* stream) {
  // the size check comes first: it touches no device state
  const size_t need = nsa_sel_dkdv_workspace(B, Hkv, T, S, block_size, chunk);
  NSA_CHECK(need > 0, NSA_ERR_SHAPE);
  NSA_CHECK(need <= kSelScratchBytes, NSA_ERR_WORKSPACE);
  void* ws = nullptr;
  const int rc = scratch_on_stream_device((hipStream_t)stream, &ws);
  if (rc != NSA_OK) return rc;
  return nsa_sel_dkdv(q, k, v, kt, dout, coff, dot, q_of_block, packed, block_offsets, pair_count, dk, dv, nullptr,
                      0, dq_part, ws, kSelScratchBytes, B, Hq, Hkv, T, D, S, block_size, chunk, dtype, stream);
}

}  // extern "C"
