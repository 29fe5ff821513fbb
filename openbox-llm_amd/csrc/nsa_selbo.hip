// Block-outer selection forward and the partial merges of the selection
// branch (the role of the reference's FSA path, nsa_selection_kernel.py:232-365
// and nsa_selection_backward.py:278-334, with the partial buffers in bf16 /
// the input dtype and the merges done by dedicated kernels).
//
// Work items are (selected block, chunk of the queries that selected it) from
// the block -> query CSR built with pack_slot (entries (t << sel_slot_bits(S)) | s).  One wave per
// item holds 64 keys of the block in registers -- K rows as the A operand of
// S^T = K Q^T, V^T as the A operand of O^T = V^T P^T -- and streams the item's
// queries two at a time (32 rows = two queries x 16 heads) through LDS.  For
// every (query, slot, pass) it writes the block-local softmax result: the
// unnormalised output O_j = sum_k p_k v_k (p_k = exp2(s_k - m_j)) in the
// input dtype and (m_j, l_j = sum_k p_k), m in log2 units.  k_sel_merge combines the partials of each query into o and lse;
// k_sel_dq_reduce sums the dQ partials written by the dK/dV kernel.
#include "nsa_items.h"
#include "nsa_launch.h"
#include "nsa_tile32.h"

namespace nsa {

constexpr float kNegInfS = -__builtin_inff();

// one 16-byte chunk of a partial row, as a non-temporal store: the rows are
// written whole (16 lanes a row) and read once by a later launch, so they
// need not stay cached (fwd 3.17 -> 3.06 ms at c3).  The dK/dV's dQ partial
// stores are not whole rows per instruction: non-temporal there, their
// partial lines reach memory unmerged (7.4 instead of 5.1 ms).
__device__ __forceinline__ void part_store(f16* p, const f16x8& v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}

// query tiles in flight per wave of k_sel_fwd_bo: three at D = 128 (one wave
// per SIMD by registers, so the stages are what keeps loads in flight: 1-1.5%
// faster than two at c3 and c5), two below (more waves fit, and a third stage
// would cost one of them its LDS)
template <int D> constexpr int fwd_bo_stages() { return D == 128 ? 3 : 2; }

// Loads of one 2-query Q tile into a natural-order row stage, issued by the
// one wave of the workgroup.  Q is packed per query, [B, Hkv, T, G, D]: the
// group's heads of one query are contiguous.  Per load a 32-bit byte offset
// below query A's rows (prepared once per head chunk) plus, for query B's
// rows, a wave-uniform distance.  Heads past the group read the group's last
// head (finite rows whose output is never stored).
template <typename T, int D> struct FwdIssuer {
  using C = Tile32<T, D>;
  static constexpr int LPT = C::ROW_CHUNKS / 64;   // loads per tile
  uint32_t off[LPT];
  uint32_t qsel;   // bit j: load j's row belongs to query B

  __device__ __forceinline__ void prepare(int grem, int lane) {
    qsel = 0;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int r, cc;
      nrow_chunk<T, D>(j * 64 + lane, r, cc);
      const int hd = (r & 15) < grem ? (r & 15) : grem - 1;
      off[j] = (uint32_t)((hd * D + cc * C::EPC) * sizeof(T));
      qsel |= (uint32_t)(r >> 4) << j;
    }
  }
  // qbh: the packed Q of the (b, hkv) and head chunk at query 0; rows are
  // addressed upward from the lower of the two queries
  __device__ __forceinline__ void issue(T* stage, const T* qbh, int tA, int tB, int G) const {
    const PairRows pr = pair_rows(tA, tB, (uint32_t)(G * D * sizeof(T)));
    const T* qa = qbh + (int64_t)pr.t0 * G * D;
#pragma unroll
    for (int j = 0; j < LPT; ++j)
      lds_dma16_sbase(qa, off[j] + (((qsel >> j) & 1u) ? pr.dB : pr.dA), (char*)stage + 1024 * j);
  }
};

// Loads of a tile of QPT = floor(32 / G) entries for groups of G <= 10 heads
// (a 2-query tile would leave 32 - 2 G rows empty): row r = q G + g is entry
// q's head g; rows from QPT G on read entry 0's head 0 (finite rows whose
// output is never stored).  Per load a 32-bit byte offset of the head and
// column (prepared once) plus t G D elements of the entry's query, read per
// lane from the item's entries.
template <typename T, int D> struct FwdIssuerGP {
  using C = Tile32<T, D>;
  static constexpr int LPT = C::ROW_CHUNKS / 64;   // loads per tile
  uint32_t off[LPT];
  int qj[LPT];   // entry (in the tile) of load j's row

  __device__ __forceinline__ void prepare(int G, int QPT, int lane) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int r, cc;
      nrow_chunk<T, D>(j * 64 + lane, r, cc);
      const bool real = r < QPT * G;
      qj[j] = real ? r / G : 0;
      const int g = real ? r % G : 0;
      off[j] = (uint32_t)((g * D + cc * C::EPC) * (int)sizeof(T));
    }
  }
  // qg: the packed Q of the (b, hkv) at query 0; t_of(i): query of entry i
  // of the item (-1 past its end); e0: the tile's first entry
  template <typename TOf>
  __device__ __forceinline__ void issue(T* stage, const T* qg, uint32_t rowbytes, int e0, TOf t_of) const {
    const int t0 = __builtin_amdgcn_readfirstlane(t_of(e0));   // a tile's first entry exists
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      int t = t_of(e0 + qj[j]);
      t = t >= 0 ? t : t0;
      lds_dma16_sbase(qg, (uint32_t)t * rowbytes + off[j], (char*)stage + 1024 * j);
    }
  }
};

// vector-memory stores of one tile's partials per wave (a lower bound:
// float tiles and D < 32 count none, which only lengthens the waits): D / 16
// staged row stores and the row statistics
template <typename T, int D>
constexpr int fwd_bo_stores() {
  return (sizeof(T) == 2 && D >= 32) ? D / 16 + 1 : 0;
}

// GP: groups of G <= 10 heads take floor(32 / G) entries per tile
// (FwdIssuerGP), the others two queries x 16 heads per head chunk.
template <typename T, int D, bool GP>
__global__ __launch_bounds__(64) void k_sel_fwd_bo(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ vt, const int32_t* __restrict__ q_of_block,
                                                   const int4* __restrict__ items,
                                                   int32_t* __restrict__ n_items, PartT<T>* __restrict__ opart,
                                                   float2* __restrict__ mlpart, int Hq, int Hkv, int T_, int S,
                                                   int n_blk, int L, int Lp, int nsub, float sl2) {
  using C = Tile32<T, D>;
  constexpr int KS = C::KS, DT = C::DT;
  constexpr int NST = fwd_bo_stages<D>();
  constexpr int LT = FwdIssuer<T, D>::LPT;
  constexpr int NSW = fwd_bo_stores<T, D>();
  static_assert((NST - 1) * (LT + NSW) < 64, "in-flight operations exceed the vmcnt range");
  __shared__ __align__(16) T sQ[NST][C::ROW_ELEMS];
  __shared__ int32_t sent[kSelItemMax];   // the item's CSR entries
  // the tile's output rows, staged so that they leave as whole rows (bf16);
  // 16-byte chunk c of row r sits at chunk c ^ (r % CPR)
  constexpr int CPR = D * (int)sizeof(T) / 16;
  __shared__ __align__(16) T sO[sizeof(T) == 2 ? 32 * D : 8];
  __shared__ int64_t srow[GP ? 32 : 1];   // GP: each tile row's partial row (element offset / D), -1: none
  const int lane = threadIdx.x, h = lane >> 5, n = lane & 31;
  const int G = Hq / Hkv, NHC = (G + 15) / 16;
  const int NS = S * nsub;
  const int sbits = sel_slot_bits(S);
  const int ni = *n_items;
  __shared__ int next_slot;
  for (int it = blockIdx.x; it < ni * nsub; it = next_item(n_items + 1, &next_slot)) {
    const int4 item = items[it / nsub];
    const int pass = it % nsub;
    const int bh = item.x / n_blk, j = item.x % n_blk;
    const int b = bh / Hkv, hkv = bh % Hkv;
    const int kbase = j * L + kSelPass * pass;
    const int kend = j * L + L < T_ ? j * L + L : T_;
    const int beg = item.y, cnt = item.z - item.y;
    // the item's entries go to LDS once: a global load per tile would be
    // waited for with every tile load in flight
    for (int i = lane; i < cnt; i += 64) sent[i] = q_of_block[beg + i];
    // block keys: K rows and V^T rows, both in perm32 order and in registers
    // (the V^T order makes each lane's outputs 8 consecutive d: 16-byte stores)
    Frag<T> kf[2][KS], vf[DT][4];
    const T* kb_ = k + (int64_t)bh * T_ * D;
    const T* vtb = vt + (int64_t)bh * D * Lp;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int key = kbase + 32 * mt + perm32(n);
      const int ks = key < kend ? key : j * L;   // finite stand-in for keys past the block
#pragma unroll
      for (int s = 0; s < KS; ++s) kf[mt][s].load(kb_ + (int64_t)ks * D + 16 * s + 8 * h);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int d = 32 * dt + perm32(n);
        int c0 = kbase + 16 * kk + 8 * h;
        c0 = c0 < Lp - 8 ? c0 : Lp - 8;
        if (D % 32 == 0 || d < D)
          vf[dt][kk].load(vtb + (int64_t)d * Lp + c0);
        else
          vf[dt][kk].zero();
      }
    // complete these loads before the walk, whose loads the compiler does not
    // see (a wait it placed inside the loop would also drain the tiles)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int s = 0; s < KS; ++s) settle(kf[mt][s]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) settle(vf[dt][kk]);
    // 16-bit inputs: one power-of-two scale s for every partial of this wave.
    // With p <= 1 (each tile's own row maximum) a partial is bounded by
    // |O_j| <= l_j max|v| <= 64 max|v| over the keys that exist, so s (1
    // below 2^15) keeps O_j / s in fp16's range.  p is divided by s inside
    // its exponent: the MFMAs then give O_j / s and l_j / s, and m_j + log2 s
    // records it.
    float lgs = 0.0f;
    if constexpr (sizeof(T) == 2) {
      float vmax = 0.0f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int c0 = kbase + 16 * kk + 8 * h;   // keys c0 .. c0 + 7 (past Lp - 8 only keys >= kend)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (c0 + i < kend) vmax = fmaxf(vmax, fabsf(to_f32(vf[dt][kk].elem(i))));
        }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o, kWave));
      const float psc = f16s_row_scale(fminf(64.0f * vmax, 3.0e38f));
      lgs = (float)((int)((__float_as_uint(psc) >> 23) & 0xffu) - 127);
    }
    __syncthreads();   // sent written
    const int QPT = GP ? 32 / G : 2;   // entries per tile
    const int ntile = (cnt + QPT - 1) / QPT;
    const int total = ntile * NHC;
    auto entry = [&](int i, int& t, int& s) {
      if (i < cnt) {
        const int v = sent[i];
        t = v >> sbits;
        s = v & ((1 << sbits) - 1);
      } else {
        t = -1;
        s = 0;
      }
    };
    auto t_of = [&](int i) {
      int t, s_;
      entry(i, t, s_);
      return t;
    };
    const int64_t qgrow = ((int64_t)b * Hkv + hkv) * T_ * G;   // packed row of query 0, head 0
    FwdIssuer<T, D> iss;
    FwdIssuerGP<T, D> issg;
    int pix = 0, phc = 0, pti = 0;   // next tile to request
    if constexpr (GP)
      issg.prepare(G, QPT, lane);
    else
      iss.prepare(G, lane);
    auto request = [&](T* stage) {
      if constexpr (GP) {
        issg.issue(stage, q + qgrow * D, (uint32_t)(G * D * (int)sizeof(T)), QPT * pti, t_of);
        ++pix;
        if (++pti == ntile) pti = 0;   // one head chunk
      } else {
        int tA, sA, tB, sB;
        entry(2 * pti, tA, sA);
        entry(2 * pti + 1, tB, sB);
        const int64_t qrow0 = qgrow + phc * 16;   // packed row of query 0, the chunk's first head
        iss.issue(stage, q + qrow0 * D, __builtin_amdgcn_readfirstlane(tA), __builtin_amdgcn_readfirstlane(tB),
                  G);
        ++pix;
        if (++pti == ntile) {
          pti = 0;
          if (++phc < NHC) iss.prepare(G - phc * 16, lane);
        }
      }
    };
    // GP: this lane's row n is entry n / G of the tile, head n % G (none from QPT G on)
    const int pq = GP ? n / G : 0, pg = GP ? n % G : 0;
    const bool preal = GP && n < QPT * G;
#pragma unroll
    for (int p = 0; p < NST; ++p)
      if (p < total) request(sQ[p]);
    for (int ix = 0; ix < total; ++ix) {
      // tile ix is complete once at most the younger tiles' loads and the
      // stores of the tiles since its request are outstanding
      if (ix + NST - 1 < total)
        vm_wait_steps<(NST - 1) * LT, NSW, NST - 1>(ix);
      else
        vm_wait<0>();
      __syncthreads();
      const T* tile = sQ[ix % NST];
      const int hc = ix / ntile, ti = ix % ntile;
      // this lane's row: query t, partial slot, head g; tlow: the tile's earliest query
      int t, slot, g, tlow;
      int tA = -1, sA = 0, tB = -1, sB = 0;
      if constexpr (GP) {
        int tl, sl;
        entry(QPT * ti + pq, tl, sl);
        t = preal ? tl : -1;
        slot = sl * nsub + pass;
        g = pg;
        tlow = 0x7fffffff;
        for (int e = 0; e < QPT; ++e) {
          const int te = __builtin_amdgcn_readfirstlane(t_of(QPT * ti + e));
          if (te < 0) break;   // entries past the item's end are the tile's last
          tlow = te < tlow ? te : tlow;
        }
      } else {
        entry(2 * ti, tA, sA);
        entry(2 * ti + 1, tB, sB);
        t = n < 16 ? tA : tB;   // query t, head hc*16 + (n & 15)
        slot = (n < 16 ? sA : sB) * nsub + pass;
        g = hc * 16 + (n & 15);
        const int utA = __builtin_amdgcn_readfirstlane(tA), utB = __builtin_amdgcn_readfirstlane(tB);
        tlow = utB >= 0 && utB < utA ? utB : utA;
      }
      const bool rok = t >= 0 && g < G;
      Frag<T> qb[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) lds_nrow_frag<T, D>(qb[s], tile, n, h, s);
      f32x16 st[2];
      st[0] = zero16();
      st[1] = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        mma32(st[0], kf[0][s], qb[s]);
        mma32(st[1], kf[1][s], qb[s]);
      }
      // raw scores; the scale (> 0) is applied to the row maximum and inside
      // the exponent's fma.  Tiles whose 64 keys all exist and precede every
      // query of the tile need no per-element mask (the earliest query
      // decides; the entries' order is not relied on).
      if (!(kbase + 64 <= kend && kbase + 63 <= tlow)) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kbase + 32 * mt + acc_elem(h, r);
            st[mt][r] = (key < kend && key <= t) ? st[mt][r] : kNegInfS;
          }
      }
      float mr = kNegInfS;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mr = fmaxf(mr, st[mt][r]);
      mr = fmaxf(mr, __shfl_xor(mr, 32, kWave));
      const float mx = mr == kNegInfS ? kNegInfS : mr * sl2;
      const float ms = (mx == kNegInfS ? 0.0f : mx) + lgs;
      float ps = 0.0f;
      Frag<T> pf[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          p[r] = fast_exp2(st[mt][r] * sl2 - ms);
          ps += p[r];
        }
        pf[2 * mt].set(p);
        pf[2 * mt + 1].set(p + 8);
      }
      const float lt = ps + __shfl_xor(ps, 32, kWave);
      f32x16 acc[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        acc[dt] = zero16();
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) mma32(acc[dt], vf[dt][kk], pf[kk]);
      }
      // refill the stage once its reads are complete
      lds_reads_done();
      if (pix < total) request(sQ[ix % NST]);
      // the partial is the unnormalised block-local output O_j = sum p v; the
      // merges weight it by exp2(m_j - M) and its l_j by the same
      if constexpr (sizeof(T) == 2) {
        // stage the rows (register r of lane half h holds d = 32 dt +
        // acc_elem(h, r)), then store them as whole rows: 64 lanes write 4
        // rows of 256 B per instruction.  A row that does not exist takes the
        // place of row 0 (always a real row: query A, first head of the
        // chunk) and rewrites its bytes, so every store instruction issues.
        static_assert(IsF16<PartT<T>>::value, "16-bit inputs keep fp16 partials");
        wave_fence();   // the previous tile's rows are read out
        // GP: each row's partial row; a row that does not exist: -1
        if constexpr (GP)
          if (h == 0) srow[n] = rok ? (((int64_t)bh * T_ + t) * NS + slot) * G + g : -1;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int c = 4 * dt + 2 * hf + h;
            if (D % 32 == 0 || c < CPR) {
              f16x8 v;
#pragma unroll
              for (int i = 0; i < 8; ++i) v[i] = (f16)acc[dt][8 * hf + i];
              *reinterpret_cast<f16x8*>(sO + (n * CPR + (c ^ (n % CPR))) * 8) = v;
            }
          }
        wave_fence();
        constexpr int RPI = 64 / CPR;   // rows per store instruction
        const int c = lane % CPR, rl = lane / CPR;
        if constexpr (GP) {
          // row r of the tile goes to its own partial row.  A row that does not
          // exist rewrites row 0's bytes (row 0: the tile's first entry, head 0,
          // always exists), so every store instruction issues.
          const int64_t r0 = srow[0];
#pragma unroll
          for (int i = 0; i < 32 / RPI; ++i) {
            const int r = RPI * i + rl;
            const int64_t ro = srow[r];
            const int rr = ro >= 0 ? r : 0;
            const f16x8 v = *reinterpret_cast<const f16x8*>(sO + (rr * CPR + (c ^ (rr % CPR))) * 8);
            part_store(opart + (ro >= 0 ? ro : r0) * D + 8 * c, v);
          }
        } else {
          // rows 0-15: query A, rows 16-31: query B, each 16 heads of G D
          // contiguous from the (query, slot) row base.  Rows that do not
          // exist repeat an existing row's bytes: a missing query B those of
          // query A, a head past G head 0 of its query.  Every store
          // instruction then issues, and for D >= 32 each one stays in one
          // query's rows, so its base address is uniform.
          const int uA = __builtin_amdgcn_readfirstlane(tA), uB = __builtin_amdgcn_readfirstlane(tB);
          const int usA = __builtin_amdgcn_readfirstlane(sA), usB = __builtin_amdgcn_readfirstlane(sB);
          PartT<T>* baseA = opart + ((((int64_t)bh * T_ + uA) * NS + usA * nsub + pass) * G + hc * 16) * D;
          PartT<T>* baseB =
              uB >= 0 ? opart + ((((int64_t)bh * T_ + uB) * NS + usB * nsub + pass) * G + hc * 16) * D : baseA;
          const int grem = G - hc * 16;   // heads of the chunk that exist
          if (uB >= 0 && grem >= 16) {
            // every row exists: the row and its base are fixed per instruction
#pragma unroll
            for (int i = 0; i < 32 / RPI; ++i) {
              const int r = RPI * i + rl;
              const f16x8 v = *reinterpret_cast<const f16x8*>(sO + (r * CPR + (c ^ (r % CPR))) * 8);
              PartT<T>* dst = (RPI * i < 16 ? baseA : baseB) + ((r & 15) * D + 8 * c);
              part_store(dst, v);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 32 / RPI; ++i) {
              const int r = RPI * i + rl;
              int rr = uB < 0 && r >= 16 ? r - 16 : r;
              rr = (rr & 15) < grem ? rr : rr & 16;
              const f16x8 v = *reinterpret_cast<const f16x8*>(sO + (rr * CPR + (c ^ (rr % CPR))) * 8);
              PartT<T>* dst = (r < 16 ? baseA : baseB) + ((rr & 15) * D + 8 * c);
              part_store(dst, v);
            }
          }
        }
        if (rok && h == 0) {
          const int64_t prow = (((int64_t)bh * T_ + t) * NS + slot) * G + g;
          // O_j / s and l_j / s (p came out divided by s) with m_j + log2 s
          mlpart[prow] = make_float2(mx == kNegInfS ? mx : mx + lgs, lt);
        }
      } else if (rok) {
        const int64_t prow = (((int64_t)bh * T_ + t) * NS + slot) * G + g;
        PartT<T>* orow = opart + prow * D;
        // register r of lane half h holds d = 32 dt + acc_elem(h, r)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int d = 32 * dt + 16 * hf + 8 * h;
            float y[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = acc[dt][8 * hf + i];
            if (D % 32 == 0 || d < D) store8(orow + d, y);
          }
        if (h == 0) mlpart[prow] = make_float2(mx, lt);
      }
    }
    vm_wait<0>();      // the walk's stores and loads are done before sent and sQ are reused
    __syncthreads();
  }
}

static inline int grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

// Both reductions below take one thread per 8 elements of a row, rows ordered
// (b, hkv, t, g) so that a wave reads contiguous partial rows.  Every slot's
// partial is loaded -- the buffers hold all NS slots of a row, and a slot
// without a pair was never written -- kSlotBatch at a time, with all loads of
// a batch issued together and none of their addresses depending on the block
// indices; a slot that does not count is then replaced by zeros (bit for bit)
// and weight 0, so whatever an unwritten slot holds never reaches a result.
constexpr int kSlotBatch = 16;

// o[row] = sum_slots exp2(m - M) O_slot / sum exp2(m - M) l over the valid
// slots, lse = (M + log2 L) ln 2, with a running maximum M across batches.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_sel_merge(const int32_t* __restrict__ idx, const PartT<T>* __restrict__ opart,
                                                   const float2* __restrict__ mlpart, T* __restrict__ o,
                                                   float* __restrict__ lse, int Hq, int Hkv, int T_, int S, int n_csr,
                                                   int L, int nsub, int64_t total, float* __restrict__ o32) {
  constexpr int NC = D / 8;
  const int G = Hq / Hkv, NS = S * nsub;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % NC);
    int64_t r = e / NC;
    const int g = (int)(r % G);
    r /= G;
    const int t = (int)(r % T_);
    const int64_t bh = r / T_;
    const int32_t* irow = idx + (bh * T_ + t) * S;
    const int64_t pbase = (bh * T_ + t) * NS;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float M = kNegInfS, Ls = 0.0f;
    for (int s0 = 0; s0 < NS; s0 += kSlotBatch) {
      float2 ml[kSlotBatch];
      Raw8<PartT<T>> x[kSlotBatch];
      bool ok[kSlotBatch];
      int jv[kSlotBatch];
#pragma unroll
      for (int k = 0; k < kSlotBatch; ++k) {
        const int sl = s0 + k < NS ? s0 + k : NS - 1;
        const int64_t pr = (pbase + sl) * G + g;
        jv[k] = irow[sl / nsub];
        ml[k] = mlpart[pr];
        x[k].load(opart + pr * D + 8 * c);
      }
      float bm = M;
#pragma unroll
      for (int k = 0; k < kSlotBatch; ++k) {
        ok[k] = (s0 + k < NS) && sel_slot_valid(jv[k], n_csr, L, t) && ml[k].y > 0.0f;
        bm = ok[k] ? fmaxf(bm, ml[k].x) : bm;
      }
      if (bm == kNegInfS) continue;   // nothing valid yet
      const float rs = M == kNegInfS ? 0.0f : fast_exp2(M - bm);
      Ls *= rs;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= rs;
#pragma unroll
      for (int k = 0; k < kSlotBatch; ++k) {
        // the partial is unnormalised; a slot that does not count was maybe
        // never written, so nothing of it (not even 0 x its l) is used
        const float wk = ok[k] ? fast_exp2(ml[k].x - bm) : 0.0f;
        x[k].keep_if(ok[k]);
        Ls += ok[k] ? wk * ml[k].y : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += wk * x[k].get(i);
      }
      M = bm;
    }
    const int64_t orow = (((bh / Hkv) * Hq + (bh % Hkv) * G + g) * T_ + t);
    const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= inv;
    if (o32 != nullptr)
      store8(o32 + orow * D + 8 * c, acc);
    else
      store8(o + orow * D + 8 * c, acc);
    if (c == 0) lse[orow] = Ls > 0.0f ? (M + __log2f(Ls)) * kLn2 : kLseEmpty;
  }
}

// dq_out[row] = (dq_acc[row] or 0) + sum over the valid slots of dqpart
// (already scaled), written in the input dtype.
template <typename T, int D>
__global__ __launch_bounds__(256) void k_sel_dq_reduce(const int32_t* __restrict__ idx, const T* __restrict__ dqpart,
                                                       const float* __restrict__ dq_acc, T* __restrict__ dq_out,
                                                       int Hq, int Hkv, int T_, int S, int n_csr, int L, int nsub,
                                                       int64_t total) {
  constexpr int NC = D / 8;
  const int G = Hq / Hkv, NS = S * nsub;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % NC);
    int64_t r = e / NC;
    const int g = (int)(r % G);
    r /= G;
    const int t = (int)(r % T_);
    const int64_t bh = r / T_;
    const int32_t* irow = idx + (bh * T_ + t) * S;
    const int64_t pbase = (bh * T_ + t) * NS;
    const int64_t orow = (((bh / Hkv) * Hq + (bh % Hkv) * G + g) * T_ + t);
    float acc[8];
    if (dq_acc != nullptr) {
      load8(dq_acc + orow * D + 8 * c, acc);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    }
    for (int s0 = 0; s0 < NS; s0 += kSlotBatch) {
      Raw8<T> x[kSlotBatch];
      int jv[kSlotBatch];
#pragma unroll
      for (int k = 0; k < kSlotBatch; ++k) {
        const int sl = s0 + k < NS ? s0 + k : NS - 1;
        jv[k] = irow[sl / nsub];
        x[k].load(dqpart + ((pbase + sl) * G + g) * D + 8 * c);
      }
#pragma unroll
      for (int k = 0; k < kSlotBatch; ++k) {
        x[k].keep_if((s0 + k < NS) && sel_slot_valid(jv[k], n_csr, L, t));
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += x[k].get(i);
      }
    }
    store8(dq_out + orow * D + 8 * c, acc);
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

static inline bool sel_args_ok(int B, int Hq, int Hkv, int T, int D, int S, int block_size) {
  return B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && S >= 0 && (D == 16 || D == 32 || D == 64 || D == 128) &&
         block_size >= 16 && block_size % 16 == 0;
}

extern "C" {

int nsa_sel_partial_slots(int S, int block_size) { return S * sel_passes(block_size); }

size_t nsa_sel_fwd_bo_workspace(int B, int Hkv, int T, int S, int block_size, int chunk) {
  if (B <= 0 || Hkv <= 0 || T < 0 || S < 0 || block_size <= 0 || chunk <= 0) return 0;
  return sel_items_cap(B, Hkv, T, S, block_size, chunk) * sizeof(int4) + 256;
}

int nsa_sel_fwd_bo(const void* q, const void* k, const void* vt, const int32_t* q_of_block,
                   const int32_t* block_offsets, void* o_part, float* ml_part, void* workspace,
                   size_t workspace_bytes, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                   int dtype, void* stream) {
  NSA_CHECK(sel_args_ok(B, Hq, Hkv, T, D, S, block_size) && chunk >= 2 && chunk <= kSelItemMax, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  // the tile loads address a group's Q rows with 32-bit byte offsets
  NSA_CHECK((int64_t)(Hq / Hkv) * T * D * (dtype == NSA_BF16 ? 2 : 4) < (1ll << 32), NSA_ERR_SHAPE);
  NSA_CHECK(workspace_bytes >= nsa_sel_fwd_bo_workspace(B, Hkv, T, S, block_size, chunk), NSA_ERR_WORKSPACE);
  const int n_blk = sel_csr_blocks(T, block_size);
  if (T == 0 || S == 0 || n_blk == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const size_t cap = sel_items_cap(B, Hkv, T, S, block_size, chunk);
  int4* items = (int4*)workspace;
  int32_t* n_items = (int32_t*)((char*)workspace + cap * sizeof(int4));
  k_sel_items<<<1, 1024, 0, s>>>(block_offsets, B * Hkv * n_blk, n_blk, chunk, items, n_items);
  if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
  const int nsub = sel_passes(block_size);
  const size_t grid = cap * nsub < 8192 ? cap * nsub : 8192;
  const int Lp = padded_len(T);
  const float sl2 = (1.0f / sqrtf((float)D)) * kLog2e;
  // groups of up to 10 heads pack floor(32 / G) >= 3 entries into a tile
  const bool gp = Hq / Hkv <= kGroupPackMaxG;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16) {
      auto kern = gp ? k_sel_fwd_bo<bf16, DD, true> : k_sel_fwd_bo<bf16, DD, false>;
      kern<<<(unsigned)grid, 64, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)vt, q_of_block, items,
                                         n_items, (f16*)o_part, (float2*)ml_part, Hq, Hkv, T, S, n_blk,
                                         block_size, Lp, nsub, sl2);
    } else {
      auto kern = gp ? k_sel_fwd_bo<float, DD, true> : k_sel_fwd_bo<float, DD, false>;
      kern<<<(unsigned)grid, 64, 0, s>>>((const float*)q, (const float*)k, (const float*)vt, q_of_block, items,
                                         n_items, (float*)o_part, (float2*)ml_part, Hq, Hkv, T, S, n_blk,
                                         block_size, Lp, nsub, sl2);
    }
  });
  return nsa_launch_status();
}

int nsa_sel_merge(const int32_t* block_idx, const void* o_part, const float* ml_part, void* o, float* lse, int B,
                  int Hq, int Hkv, int T, int D, int S, int block_size, int dtype, int o_dtype, void* stream) {
  NSA_CHECK(sel_args_ok(B, Hq, Hkv, T, D, S, block_size), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(o_dtype == dtype || o_dtype == NSA_F32, NSA_ERR_DTYPE);
  float* o32 = o_dtype == NSA_F32 && dtype != NSA_F32 ? (float*)o : nullptr;
  const int64_t total = (int64_t)B * Hq * T * (D / 8);
  if (total == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int n_csr = sel_csr_blocks(T, block_size), nsub = sel_passes(block_size);
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16)
      k_sel_merge<bf16, DD><<<grid_for(total), 256, 0, s>>>(block_idx, (const f16*)o_part, (const float2*)ml_part,
                                                            o32 ? nullptr : (bf16*)o, lse, Hq, Hkv, T, S, n_csr,
                                                            block_size, nsub, total, o32);
    else
      k_sel_merge<float, DD><<<grid_for(total), 256, 0, s>>>(block_idx, (const float*)o_part,
                                                             (const float2*)ml_part, (float*)o, lse, Hq, Hkv, T, S,
                                                             n_csr, block_size, nsub, total, nullptr);
  });
  return nsa_launch_status();
}

int nsa_sel_dq_reduce(const int32_t* block_idx, const void* dq_part, const float* dq_acc, void* dq_out, int B,
                      int Hq, int Hkv, int T, int D, int S, int block_size, int dtype, void* stream) {
  NSA_CHECK(sel_args_ok(B, Hq, Hkv, T, D, S, block_size), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  const int64_t total = (int64_t)B * Hq * T * (D / 8);
  if (total == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int n_csr = sel_csr_blocks(T, block_size), nsub = sel_passes(block_size);
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16)
      k_sel_dq_reduce<bf16, DD><<<grid_for(total), 256, 0, s>>>(block_idx, (const bf16*)dq_part, dq_acc,
                                                                (bf16*)dq_out, Hq, Hkv, T, S, n_csr, block_size,
                                                                nsub, total);
    else
      k_sel_dq_reduce<float, DD><<<grid_for(total), 256, 0, s>>>(block_idx, (const float*)dq_part, dq_acc,
                                                                 (float*)dq_out, Hq, Hkv, T, S, n_csr, block_size,
                                                                 nsub, total);
  });
  return nsa_launch_status();
}

}  // extern "C"
