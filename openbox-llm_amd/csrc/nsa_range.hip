// Range branches of NSA (sliding window, compression over pooled keys):
// forward and dQ, LDS-tiled on 32x32 MFMAs.
//
// Rows of the attention are (query, head) pairs: the 16 heads of one GQA head
// chunk of a query form 16 consecutive rows, so a 32-row MFMA tile holds two
// queries.  A wave owns NT such tiles (2*NT consecutive queries) and a
// workgroup of four waves owns 8*NT consecutive queries of one KV head chunk.
// Groups of G < 16 heads number their rows t G + g instead and take 32
// consecutive rows per wave (flat rows, range_rows).
// The workgroup walks the union of its queries' visible key range in 32-key
// tiles; each tile of K (row-major) and V^T (or K, V and K^T for dQ) is
// staged once in LDS by direct global -> LDS loads, double-buffered, and read
// by all four waves.
//
//   forward:  S^T = K Q^T (keys on M, rows on N), online softmax per row,
//             O^T += V^T P^T with P^T taken straight from the S^T accumulator
//   dQ:       S^T = K Q^T, dP^T = V dO^T, dS^T = P^T (dP^T - delta),
//             dQ^T += K^T dS^T
// Key rows of K / V are read through perm32 so that the accumulator registers
// line up with the next contraction's operand slots (nsa_tile32.h).
#include "nsa_items.h"
#include "nsa_launch.h"
#include "nsa_tile32.h"

namespace nsa {

struct RangeMap {
  int b, hkv, hc, G, NHC;
};

__device__ __forceinline__ RangeMap range_map(int64_t r, int Hq, int Hkv) {
  RangeMap m;
  m.G = Hq / Hkv;
  m.NHC = (m.G + 15) / 16;
  m.hc = (int)(r % m.NHC);
  const int bh = (int)(r / m.NHC);
  m.b = bh / Hkv;
  m.hkv = bh % Hkv;
  return m;
}

// visible key range [lo, hi] of query t (hi < lo: none)
__device__ __forceinline__ void visible_range(int mode, int t, int Lk, int window, int cl, int cd, int& lo,
                                              int& hi) {
  if (mode == NSA_MODE_WINDOW) {
    lo = t - window + 1 > 0 ? t - window + 1 : 0;
    hi = t < Lk - 1 ? t : Lk - 1;
  } else {
    lo = 0;
    hi = t >= cl - 1 ? (t - cl + 1) / cd : -1;
    hi = hi < Lk - 1 ? hi : Lk - 1;
  }
}

// Workgroup / wave query and key ranges of a range launch.
struct RangeSpan {
  int klo, khi;     // union of visible keys of the workgroup's queries
  int wlo, whi;     // union for this wave's queries
};

__device__ __forceinline__ RangeSpan range_span(int mode, int tb0, int qpb, int tw0, int qpw, int T_, int Lk,
                                                int window, int cl, int cd) {
  RangeSpan s;
  int lo, hi;
  const int tb1 = tb0 + qpb - 1 < T_ - 1 ? tb0 + qpb - 1 : T_ - 1;
  visible_range(mode, tb0, Lk, window, cl, cd, s.klo, hi);
  visible_range(mode, tb1, Lk, window, cl, cd, lo, s.khi);
  if (tw0 < T_) {
    const int tw1 = tw0 + qpw - 1 < T_ - 1 ? tw0 + qpw - 1 : T_ - 1;
    visible_range(mode, tw0, Lk, window, cl, cd, s.wlo, hi);
    visible_range(mode, tw1, Lk, window, cl, cd, lo, s.whi);
  } else {
    s.wlo = 0;
    s.whi = -1;
  }
  return s;
}

// Keys visible to every valid query of a wave: a tile inside [lo, hi] needs no
// per-element mask.
struct FullSpan {
  int lo, hi;
};

__device__ __forceinline__ FullSpan full_span(int mode, int tw0, int qpw, int T_, int Lk, int window, int cl,
                                              int cd) {
  FullSpan f;
  if (tw0 >= T_) {
    f.lo = 0;
    f.hi = 1 << 30;   // no valid row: nothing to mask
    return f;
  }
  const int tw1 = tw0 + qpw - 1 < T_ - 1 ? tw0 + qpw - 1 : T_ - 1;
  int lo0, hi0, lo1, hi1;
  visible_range(mode, tw0, Lk, window, cl, cd, lo0, hi0);
  visible_range(mode, tw1, Lk, window, cl, cd, lo1, hi1);
  f.lo = lo1 > lo0 ? lo1 : lo0;   // lo and hi are non-decreasing in t
  f.hi = hi0 < hi1 ? hi0 : hi1;
  return f;
}

// Rows of a range launch.  Head-chunk rows (groups of 16 or more heads): a
// workgroup owns 8 NT consecutive queries of one head chunk and a wave 2 NT of
// them; row n of a wave's tile nt is query tw0 + 2 nt + (n >> 4), head
// hc 16 + (n & 15) of the group.  Flat rows (groups of G < 16 heads, NT = 1):
// the rows (t, g) of one (b, hkv) are numbered t G + g, a workgroup owns 128
// consecutive ones and a wave 32 (row n: rw0 + n), so only the sequence's last
// tile has empty rows where a head chunk would leave 16 - G of every 16 empty.
// qpb / qpw count the queries the workgroup's / wave's rows touch; a wave past
// the last row gets tw0 = T (no valid row).
struct RangeRows {
  int tb0, qpb, tw0, qpw, rw0;
};
template <bool FLAT, int NT>
__device__ __forceinline__ bool range_rows(RangeRows& r, int qt, int w, int G, int T_) {
  if constexpr (FLAT) {
    static_assert(NT == 1, "flat rows: one 32-row tile per wave");
    const int nrow = T_ * G;
    const int rb0 = qt * 128;
    if (rb0 >= nrow) return false;
    r.tb0 = rb0 / G;
    r.qpb = (rb0 + 127 < nrow ? rb0 + 127 : nrow - 1) / G - r.tb0 + 1;
    r.rw0 = rb0 + 32 * w;
    if (r.rw0 < nrow) {
      r.tw0 = r.rw0 / G;
      r.qpw = (r.rw0 + 31 < nrow ? r.rw0 + 31 : nrow - 1) / G - r.tw0 + 1;
    } else {
      r.tw0 = T_;
      r.qpw = 1;
    }
  } else {
    r.tb0 = qt * 8 * NT;
    if (r.tb0 >= T_) return false;
    r.qpb = 8 * NT;
    r.tw0 = r.tb0 + w * 2 * NT;
    r.qpw = 2 * NT;
    r.rw0 = 0;
  }
  return true;
}
// query and head (within the group) of row n of a wave's tile nt
template <bool FLAT>
__device__ __forceinline__ void range_row(const RangeRows& r, const RangeMap& mp, int nt, int n, int& t, int& g) {
  if constexpr (FLAT) {
    const int R = r.rw0 + n;
    t = R / mp.G;
    g = R - t * mp.G;
  } else {
    t = r.tw0 + 2 * nt + (n >> 4);
    g = mp.hc * 16 + (n & 15);
  }
}
// query tiles of a range launch per (b, hkv, head chunk)
__host__ __device__ inline int range_qtiles(bool flat, int T, int G, int NT) {
  return flat ? (T * G + 127) / 128 : (T + 8 * NT - 1) / (8 * NT);
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// Optional extra outputs of a forward launch.  q_packed: the Q rows the
// launch loads, also stored in the nsa_pack_heads layout.  opart: the launch
// finishes the rows of the gated layer (as the last branch, the window): it
// merges the selection partials of nsa_sel_fwd_bo for its rows into o_sel /
// lse_sel (the role of nsa_sel_merge) and blends the three branches through
// the gate into out (the role of nsa_gate_fwd), each from the same rounded
// branch outputs the separate kernels would read.
// TO is the type of the branch outputs (o, o_sel, o_cmp): the input type T,
// float when the caller keeps them unrounded for the backward's row dots, or
// f16 for the NSA_F16S form (fp16 rows, a float32 scale per row after them:
// o_scale, o_sel_scale, o_cmp_scale).
template <typename T, typename TO> struct FwdExtras {
  T* q_packed;             // [B][Hkv][T][G][D] (nullable)
  const PartT<T>* opart;   // [B][Hkv][T][NS][G][D] unnormalised block-local outputs O_j = sum p v
  const float2* ml;        // [B][Hkv][T][NS][G] (m_j [log2 units], l_j)
  const int32_t* idx;      // [B][Hkv][T][S] selected blocks
  TO* o_sel;               // [B][Hq][T][D]
  float* lse_sel;          // [B][Hq][T]
  const TO* o_cmp;         // [B][Hq][T][D] compression output
  const T* gate;           // [B][Hq][T][3] gate logits
  T* out;                  // [B][Hq][T][D]
  int S, sel_L;
  float* out32;            // nullable: out in float32 (unrounded), written instead of `out`
  float* o_scale;          // NSA_F16S row scales of this launch's o, o_sel and o_cmp
  float* o_sel_scale;
  const float* o_cmp_scale;
};

// The wave's own output rows (this branch, unnormalised acc with the row
// statistics l_, m_) go through LDS so that every row is handled in 8-element
// chunks: lane (row sub-index, chunk) per pass.
template <typename T, typename TO, int D, bool FLAT>
__device__ __forceinline__ void finish_rows(const FwdExtras<T, TO>& f, const f32x16 (&acc)[Tile32<T, D>::DT][1],
                                            float l_row, float m_row, bool any_key, bool rok, int64_t row, TO* o,
                                            float* lse, char* smem, int w, int lane, const RangeRows& rr,
                                            const RangeMap& mp, int Hq, int Hkv, int T_) {
  using C = Tile32<T, D>;
  constexpr int FIN_PITCH = D + 4;
  const int h = lane >> 5, n = lane & 31;
  const float lt = l_row + __shfl_xor(l_row, 32, kWave);
  const float inv = any_key ? 1.0f / lt : 0.0f;
  if (rok && h == 0) lse[row] = any_key ? (m_row + __log2f(lt)) * kLn2 : kLseEmpty;
  __syncthreads();   // the key stages are free
  float* fin = reinterpret_cast<float*>(smem) + w * 32 * FIN_PITCH;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * dt + 8 * g4 + 4 * h;
      if (D % 32 == 0 || d < D)
        *reinterpret_cast<f32x4*>(fin + n * FIN_PITCH + d) =
            (f32x4){acc[dt][0][4 * g4], acc[dt][0][4 * g4 + 1], acc[dt][0][4 * g4 + 2], acc[dt][0][4 * g4 + 3]} *
            inv;
    }
  __syncthreads();
  constexpr int CPR = D / 8, RPI = 64 / CPR;   // 8-element chunks per row, rows per pass
  const int c8 = lane % CPR, rsub = lane / CPR;
  const int nsub = sel_passes(f.sel_L), NS = f.S * nsub, n_csr = sel_csr_blocks(T_, f.sel_L);
  const int G = mp.G;
  const int64_t bh = (int64_t)mp.b * Hkv + mp.hkv;
  for (int r0 = 0; r0 < 32; r0 += RPI) {
    const int r = r0 + rsub;
    int t, gl;   // query and head within the group
    range_row<FLAT>(rr, mp, 0, r, t, gl);
    if (t >= T_ || gl >= G) continue;
    const int64_t orow = ((int64_t)mp.b * Hq + mp.hkv * G + gl) * T_ + t;
    // the gate's other operands (compression row and logits) are loaded
    // first: their latency then overlaps the partials', not follows it
    Raw8<TO> ocr;
    ocr.load(f.o_cmp + orow * D + 8 * c8);
    const float ocs = IsF16<TO>::value ? f.o_cmp_scale[orow] : 1.0f;
    const T gr0 = f.gate[orow * 3 + 0], gr1 = f.gate[orow * 3 + 1], gr2 = f.gate[orow * 3 + 2];
    // this branch's row chunk, rounded as stored
    float ow[8];
    {
      const f32x4 a = *reinterpret_cast<const f32x4*>(fin + r * FIN_PITCH + 8 * c8);
      const f32x4 b2 = *reinterpret_cast<const f32x4*>(fin + r * FIN_PITCH + 8 * c8 + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) ow[i] = a[i], ow[4 + i] = b2[i];
      store_branch8<TO, CPR, kWholeLines<D>>(o + orow * D + 8 * c8, ow, f.o_scale + orow, c8 == 0);
    }
    // selection: merge the slot partials (running maximum over batches of 16)
    const int64_t qs = bh * T_ + t;
    const int32_t* irow = f.idx + qs * f.S;
    float acc_s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float M = -__builtin_inff(), Ls = 0.0f;
    for (int s0 = 0; s0 < NS; s0 += 16) {
      Raw8<PartT<T>> x[16];
      float2 ml[16];
      int jv[16];
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) {
        const int sl = s0 + k2 < NS ? s0 + k2 : NS - 1;
        const int64_t pr = (qs * NS + sl) * G + gl;
        jv[k2] = irow[sl / nsub];
        ml[k2] = f.ml[pr];
        x[k2].load_nt(f.opart + pr * D + 8 * c8);
      }
      bool ok[16];
      float bm = M;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) {
        ok[k2] = s0 + k2 < NS && sel_slot_valid(jv[k2], n_csr, f.sel_L, t) && ml[k2].y > 0.0f;
        bm = ok[k2] ? fmaxf(bm, ml[k2].x) : bm;
      }
      if (bm == -__builtin_inff()) continue;   // nothing valid yet
      const float rs = M == -__builtin_inff() ? 0.0f : fast_exp2(M - bm);
      Ls *= rs;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc_s[i] *= rs;
#pragma unroll
      for (int k2 = 0; k2 < 16; ++k2) {
        // the partial is unnormalised; a slot that does not count was maybe
        // never written, so nothing of it (not even 0 x its l) is used
        const float wk = ok[k2] ? fast_exp2(ml[k2].x - bm) : 0.0f;
        x[k2].keep_if(ok[k2]);
        Ls += ok[k2] ? wk * ml[k2].y : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc_s[i] += wk * x[k2].get(i);
      }
      M = bm;
    }
    const float inv_s = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc_s[i] *= inv_s;
    store_branch8<TO, CPR, kWholeLines<D>>(f.o_sel + orow * D + 8 * c8, acc_s, f.o_sel_scale + orow, c8 == 0);
    if (c8 == 0) f.lse_sel[orow] = Ls > 0.0f ? (M + __log2f(Ls)) * kLn2 : kLseEmpty;
    // gate: sigmoid-weighted sum of the three rounded branch outputs
    const float g0 = sigmoidf(to_f32(gr0));
    const float g1 = sigmoidf(to_f32(gr1));
    const float g2 = sigmoidf(to_f32(gr2));
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float oc = IsF16<TO>::value ? ocr.get(i) * ocs : ocr.get(i);
      y[i] = g0 * oc + g1 * acc_s[i] + g2 * ow[i];
    }
    if (f.out32 != nullptr)
      store8(f.out32 + orow * D + 8 * c8, y);
    else
      store8_as<kWholeLines<D>>(f.out + orow * D + 8 * c8, y);
  }
}
constexpr float kNegInf = -__builtin_inff();
constexpr float kRescale = 8.0f;   // log2 growth of a row maximum that forces a rescale

// One 32-key tile of the forward for NT row tiles.  pv_split (16-bit
// operands): P enters the PV product as two operands, its bf16 rounding and
// the remainder (about 16 significant bits instead of 8), so the stored o
// (and the backward's row dot dO . o, whose error dS = P (dP - dot) passes on
// whole to dQ and dK) carries no P rounding; the window forward uses it (at
// config 4 its dQ error fell from 1.8e-2 to 1.2e-2 for 0.06 ms a step), the
// compression forward does not (0.29 ms for no measurable gain).  mask =
// false: every key of the tile is visible to every valid row of the wave (no
// per-element test).
// The row maximum m is only moved when the tile's maximum exceeds it by more
// than kRescale (wave-uniform branch); p = exp2(s - m) <= 2^kRescale keeps the
// sum and the bf16 P operand in range, and the final 1/l normalises exactly.
template <typename T, int D, int NT, int DT = Tile32<T, D>::DT, int KS = Tile32<T, D>::KS>
__device__ __forceinline__ void fwd_tile(f32x16 (&acc)[DT][NT], float (&m_)[NT], float (&l_)[NT],
                                         const Frag<T> (&qf)[NT][KS], const T* tK, const T* tV, int kb, bool mask,
                                         const int (&lo)[NT], const int (&hi)[NT], float sl2, int n, int h,
                                         bool pv_split) {
  // all K fragments of the tile first, so the LDS reads are in flight together
  Frag<T> ka[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) lds_row_frag<T, D>(ka[s], tK, n, h, s);
  f32x16 st[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) st[nt] = zero16();
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) mma32(st[nt], ka[s], qf[nt][s]);
  // V^T fragments of the tile, issued before the softmax arithmetic
  Frag<T> va[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) lds_col_frag<T, D>(va[dt][s], tV, dt, n, h, s);
  // st holds raw scores: the scale (> 0) is applied to the row maximum and
  // inside the exponent's fma
  if (mask) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + acc_elem(h, r);
        st[nt][r] = (key >= lo[nt] && key <= hi[nt]) ? st[nt][r] : kNegInf;
      }
  }
  float mx[NT];
  bool need = false;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float v = st[nt][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) v = fmaxf(v, st[nt][r]);
    mx[nt] = fmaxf(v, __shfl_xor(v, 32, kWave)) * sl2;
    need |= mx[nt] > m_[nt] + kRescale;
  }
  if (__any(need)) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float mn = mx[nt] > m_[nt] + kRescale ? mx[nt] : m_[nt];
      const float alpha = fast_exp2(m_[nt] - mn);
      l_[nt] *= alpha;
      m_[nt] = mn;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt][nt] *= alpha;
    }
  }
  Frag<T> pf[NT][2], pl[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float p[16];
    float ps = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = fast_exp2(st[nt][r] * sl2 - m_[nt]);
      ps += p[r];
    }
    l_[nt] += ps;
    pf[nt][0].set(p);
    pf[nt][1].set(p + 8);
    if constexpr (sizeof(T) == 2) {
      if (pv_split) {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] -= to_f32(from_f32<T>(p[r]));
        pl[nt][0].set(p);
        pl[nt][1].set(p + 8);
      }
    }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) mma32(acc[dt][nt], va[dt][s], pf[nt][s]);
  if constexpr (sizeof(T) == 2) {
    if (pv_split) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) mma32(acc[dt][nt], va[dt][s], pl[nt][s]);
    }
  }
}

template <typename T, int D, int NT, typename TO, bool FLAT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_range_fwd32(int mode, const T* __restrict__ q, const T* __restrict__ k,
                                                     const T* __restrict__ vt, TO* __restrict__ o,
                                                     float* __restrict__ lse, int Hq, int Hkv, int T_, int Lk,
                                                     int Lp, int nqt, int window, int cl, int cd, float sl2,
                                                     const FwdExtras<T, TO> fin_args) {
  using C = Tile32<T, D>;
  constexpr int NST = 4;   // key tiles in flight + 1
  // one LDS buffer: the key stages during the walk, then (finishing rows)
  // each wave's float output tile [32][D + 4]
  constexpr int FIN_PITCH = D + 4;
  constexpr int STAGE_BYTES = NST * (C::ROW_ELEMS + C::COL_ELEMS) * (int)sizeof(T);
  constexpr int FIN_BYTES = 4 * 32 * FIN_PITCH * (int)sizeof(float);
  __shared__ __align__(16) char smem[STAGE_BYTES > FIN_BYTES ? STAGE_BYTES : FIN_BYTES];
  T (*sK)[C::ROW_ELEMS] = reinterpret_cast<T (*)[C::ROW_ELEMS]>(smem);
  T (*sV)[C::COL_ELEMS] = reinterpret_cast<T (*)[C::COL_ELEMS]>(smem + NST * C::ROW_ELEMS * sizeof(T));
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  // window: neighbouring query tiles (which share keys) on one XCD;
  // compression: every tile reads the same small key set and the work grows
  // with t, so tiles go out round-robin, longest first, to balance the XCDs
  const int64_t wg = mode == NSA_MODE_COMPRESS ? (int64_t)blockIdx.x : xcd_remap(blockIdx.x, gridDim.x);
  int qt = (int)(wg % nqt);
  if (mode == NSA_MODE_COMPRESS) qt = nqt - 1 - qt;   // long rows first
  const RangeMap mp = range_map(wg / nqt, Hq, Hkv);
  RangeRows rr;
  if (!range_rows<FLAT, NT>(rr, qt, w, mp.G, T_)) return;
  const int tw0 = rr.tw0;
  const RangeSpan sp = range_span(mode, rr.tb0, rr.qpb, tw0, rr.qpw, T_, Lk, window, cl, cd);
  const FullSpan fs = full_span(mode, tw0, rr.qpw, T_, Lk, window, cl, cd);
  const int bh = mp.b * Hkv + mp.hkv;
  const T* kbase = k + (int64_t)bh * Lk * D;
  const T* vtbase = vt + (int64_t)bh * D * Lp;

  Frag<T> qf[NT][C::KS];
  int lo[NT], hi[NT];
  int64_t row[NT];
  bool rok[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    int t, g;   // this lane's row: query t, head g of the group
    range_row<FLAT>(rr, mp, nt, n, t, g);
    rok[nt] = g < mp.G && t < T_;
    const int head = mp.hkv * mp.G + g;
    row[nt] = ((int64_t)mp.b * Hq + head) * T_ + t;
    const int64_t srow = ((int64_t)mp.b * Hq + (rok[nt] ? head : mp.hkv * mp.G)) * T_ + (t < T_ ? t : T_ - 1);
    visible_range(mode, t < T_ ? t : T_ - 1, Lk, window, cl, cd, lo[nt], hi[nt]);
#pragma unroll
    for (int s = 0; s < C::KS; ++s) qf[nt][s].load(q + srow * D + 16 * s + 8 * h);
    if (fin_args.q_packed != nullptr && rok[nt]) {
      T* dst = fin_args.q_packed + (((int64_t)bh * T_ + t) * mp.G + g) * D;
#pragma unroll
      for (int s = 0; s < C::KS; ++s) qf[nt][s].store(dst + 16 * s + 8 * h);
    }
  }
  float m_[NT], l_[NT];
  f32x16 acc[C::DT][NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_[nt] = kMaskScore;
    l_[nt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[dt][nt] = zero16();
  }

  const int kt0 = sp.klo & ~31;
  const int ntile = sp.khi >= sp.klo ? (sp.khi - kt0) / 32 + 1 : 0;
  // the Q fragments complete before the walk (whose loads the compiler does
  // not see: a wait it placed in the loop would drain the tiles in flight)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int s = 0; s < C::KS; ++s) settle(qf[nt][s]);
  RowTileDma<T, D, 256, false> kdma;
  ColTileDma<T, D, 256> vdma;
  kdma.init(tid);
  vdma.init(tid, Lp);
  constexpr int LT = decltype(kdma)::NL + decltype(vdma)::NL;
  // unrolled over the stages (immediate stage addresses): 1-2% faster here;
  // the dQ and the top-n walk measured no gain from it
  key_pipeline_st<NST, LT>(ntile, [&](int i, auto st) {
    kdma.request(sK[decltype(st)::value], kbase, kt0 + 32 * i, Lk, tid);
    vdma.request(sV[decltype(st)::value], vtbase, kt0 + 32 * i, tid);
  }, [&](int it, auto st) {
    const int kb = kt0 + 32 * it;
    // every wave takes every tile of the workgroup range (the waves' own ranges
    // differ by at most a few queries); tiles inside the wave's fully visible
    // span skip the per-element mask
    const bool mask = !(kb >= fs.lo && kb + 31 <= fs.hi);
    fwd_tile<T, D, NT>(acc, m_, l_, qf, sK[decltype(st)::value], sV[decltype(st)::value], kb, mask, lo, hi, sl2, n,
                       h, mode == NSA_MODE_WINDOW);
  });

  if (fin_args.opart != nullptr) {
    static_assert(NT == 1, "one 32-row tile per wave is staged");
    finish_rows<T, TO, D, FLAT>(fin_args, acc, l_[0], m_[0], lo[0] <= hi[0], rok[0], row[0], o, lse, smem, w,
                                lane, rr, mp, Hq, Hkv, T_);
    return;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float lt = l_[nt] + __shfl_xor(l_[nt], 32, kWave);
    const bool any_key = lo[nt] <= hi[nt];
    float inv = any_key ? 1.0f / lt : 0.0f;
    if constexpr (IsF16<TO>::value) {
      // NSA_F16S: the row's scale from its largest magnitude (the two lanes
      // of column n hold the row's halves)
      float amax = 0.0f;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (D % 32 == 0 || 32 * dt + 8 * (i >> 2) + 4 * h < D) amax = fmaxf(amax, fabsf(acc[dt][nt][i]));
      amax = fmaxf(amax, __shfl_xor(amax, 32, kWave)) * inv;
      const float sc = f16s_row_scale(amax);
      if (rok[nt] && h == 0) fin_args.o_scale[row[nt]] = sc;
      inv /= sc;
    }
    if (!rok[nt]) continue;
    TO* orow = o + row[nt] * D;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * h;
        if (D % 32 == 0 || d < D)
          store4(orow + d, acc[dt][nt][4 * g4] * inv, acc[dt][nt][4 * g4 + 1] * inv, acc[dt][nt][4 * g4 + 2] * inv,
                 acc[dt][nt][4 * g4 + 3] * inv);
      }
    }
    if (h == 0) lse[row[nt]] = any_key ? (m_[nt] + __log2f(lt)) * kLn2 : kLseEmpty;
  }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
// Optional second branch of a dQ launch: the window branch over keys of the
// query length, walked after the launch's compression keys into the same dQ
// accumulators (k == nullptr: none).
template <typename T> struct DqWindow {
  const T* k;
  const T* v;
  const T* kt;
  const float* lse;
  const float* dot;
  const float* rowscale;
  int Lp;
};

// One 32-key tile of dQ for NT row tiles; c = lse*log2(e) - log2(rowscale) per
// row, so P = exp2(S*sl2 - c) carries the gate weight.
template <typename T, int D, int NT, int DT = Tile32<T, D>::DT, int KS = Tile32<T, D>::KS>
__device__ __forceinline__ void dq_tile(f32x16 (&acc)[DT][NT], const Frag<T> (&qf)[NT][KS],
                                        const Frag<T> (&df)[NT][KS], const T* tK, const T* tV, const T* tKt, int kb,
                                        bool mask, const int (&lo)[NT], const int (&hi)[NT], const float (&c)[NT],
                                        const float (&dlt)[NT], float sl2, int n, int h) {
  f32x16 st[NT], pt[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    st[nt] = zero16();
    pt[nt] = zero16();
  }
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    Frag<T> a, b;
    lds_row_frag<T, D>(a, tK, n, h, s);
    lds_row_frag<T, D>(b, tV, n, h, s);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      mma32(st[nt], a, qf[nt][s]);
      mma32(pt[nt], b, df[nt][s]);
    }
  }
  // K^T fragments of the tile, issued before the dS arithmetic
  Frag<T> ka[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) lds_col_frag<T, D>(ka[dt][s], tKt, dt, n, h, s);
  Frag<T> dsf[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(st[nt][r] * sl2 - c[nt]);
    if (mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + acc_elem(h, r);
        p[r] = (key >= lo[nt] && key <= hi[nt]) ? p[r] : 0.0f;
      }
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ds[r] = p[r] * (pt[nt][r] - dlt[nt]);
    dsf[nt][0].set(ds);
    dsf[nt][1].set(ds + 8);
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) mma32(acc[dt][nt], ka[dt][s], dsf[nt][s]);
}

template <typename T, int D, int NT, bool FLAT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_range_dq32(int mode, const T* __restrict__ q, const T* __restrict__ k,
                                                    const T* __restrict__ v, const T* __restrict__ kt,
                                                    const T* __restrict__ dout, const float* __restrict__ lse,
                                                    const float* __restrict__ dot,
                                                    const float* __restrict__ rowscale, float* __restrict__ dq,
                                                    int accumulate, int Hq, int Hkv, int T_, int Lk, int Lp, int nqt,
                                                    int window, int cl, int cd, float sl2, float scale,
                                                    const T* __restrict__ sel_part, const int32_t* __restrict__ sel_idx,
                                                    T* __restrict__ dq_out, float* __restrict__ dq_out32, int S,
                                                    int sel_L, DqWindow<T> w2) {
  using C = Tile32<T, D>;
  constexpr int NST = 3;   // key tiles in flight + 1
  // one LDS buffer: the key stages during the walk, then (finishing rows)
  // each wave's float dQ tile [32][D + 4]
  constexpr int FIN_PITCH = D + 4;
  constexpr int STAGE_BYTES = NST * (2 * C::ROW_ELEMS + C::COL_ELEMS) * (int)sizeof(T);
  constexpr int FIN_BYTES = 4 * 32 * FIN_PITCH * (int)sizeof(float);
  __shared__ __align__(16) char smem[STAGE_BYTES > FIN_BYTES ? STAGE_BYTES : FIN_BYTES];
  T (*sK)[C::ROW_ELEMS] = reinterpret_cast<T (*)[C::ROW_ELEMS]>(smem);
  T (*sV)[C::ROW_ELEMS] = reinterpret_cast<T (*)[C::ROW_ELEMS]>(smem + NST * C::ROW_ELEMS * sizeof(T));
  T (*sKt)[C::COL_ELEMS] = reinterpret_cast<T (*)[C::COL_ELEMS]>(smem + 2 * NST * C::ROW_ELEMS * sizeof(T));
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const int64_t wg = mode == NSA_MODE_COMPRESS ? (int64_t)blockIdx.x : xcd_remap(blockIdx.x, gridDim.x);
  int qt = (int)(wg % nqt);
  if (mode == NSA_MODE_COMPRESS) qt = nqt - 1 - qt;   // long rows first, round-robin (as the forward)
  const RangeMap mp = range_map(wg / nqt, Hq, Hkv);
  RangeRows rr;
  if (!range_rows<FLAT, NT>(rr, qt, w, mp.G, T_)) return;
  const int tw0 = rr.tw0;
  const int bh = mp.b * Hkv + mp.hkv;

  Frag<T> qf[NT][C::KS], df[NT][C::KS];
  int64_t row[NT], srow[NT];
  int trow[NT];   // this lane's query per tile
  bool rok[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    int t, g;   // this lane's row: query t, head g of the group
    range_row<FLAT>(rr, mp, nt, n, t, g);
    const int tc = t < T_ ? t : T_ - 1;
    trow[nt] = t;
    rok[nt] = g < mp.G && t < T_;
    const int head = mp.hkv * mp.G + g;
    row[nt] = ((int64_t)mp.b * Hq + head) * T_ + t;
    srow[nt] = ((int64_t)mp.b * Hq + (rok[nt] ? head : mp.hkv * mp.G)) * T_ + tc;
#pragma unroll
    for (int s = 0; s < C::KS; ++s) {
      qf[nt][s].load(q + srow[nt] * D + 16 * s + 8 * h);
      df[nt][s].load(dout + srow[nt] * D + 16 * s + 8 * h);
    }
  }
  f32x16 acc[C::DT][NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[dt][nt] = zero16();
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int s = 0; s < C::KS; ++s) settle(qf[nt][s]), settle(df[nt][s]);
  RowTileDma<T, D, 256, false> rdma;   // K and V rows share the per-lane offsets
  rdma.init(tid);

  // one branch's walk over its keys, accumulating into acc
  auto walk = [&](int bmode, const T* k_, const T* v_, const T* kt_, const float* lse_, const float* dot_,
                  const float* rs_, int Lk_, int Lp_) {
    const RangeSpan sp = range_span(bmode, rr.tb0, rr.qpb, tw0, rr.qpw, T_, Lk_, window, cl, cd);
    const FullSpan fs = full_span(bmode, tw0, rr.qpw, T_, Lk_, window, cl, cd);
    int lo[NT], hi[NT];
    float c[NT], dlt[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int t = trow[nt];
      visible_range(bmode, t < T_ ? t : T_ - 1, Lk_, window, cl, cd, lo[nt], hi[nt]);
      const float rs = rs_ != nullptr ? rs_[srow[nt]] : 1.0f;
      c[nt] = lse_[srow[nt]] * kLog2e - __log2f(rs);
      dlt[nt] = dot_[srow[nt]];
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) asm volatile("" : "+v"(c[nt]), "+v"(dlt[nt]));
    const int kt0 = sp.klo & ~31;
    const int ntile = sp.khi >= sp.klo ? (sp.khi - kt0) / 32 + 1 : 0;
    const T* kbase = k_ + (int64_t)bh * Lk_ * D;
    const T* vbase = v_ + (int64_t)bh * Lk_ * D;
    const T* ktbase = kt_ + (int64_t)bh * D * Lp_;
    ColTileDma<T, D, 256> ktdma;
    ktdma.init(tid, Lp_);
    constexpr int LT = 2 * decltype(rdma)::NL + decltype(ktdma)::NL;
    key_pipeline<NST, LT>(ntile, [&](int i) {
      rdma.request(sK[i % NST], kbase, kt0 + 32 * i, Lk_, tid);
      rdma.request(sV[i % NST], vbase, kt0 + 32 * i, Lk_, tid);
      ktdma.request(sKt[i % NST], ktbase, kt0 + 32 * i, tid);
    }, [&](int it) {
      const int kb = kt0 + 32 * it;
      const bool mask = !(kb >= fs.lo && kb + 31 <= fs.hi);
      dq_tile<T, D, NT>(acc, qf, df, sK[it % NST], sV[it % NST], sKt[it % NST], kb, mask, lo, hi, c, dlt, sl2, n,
                        h);
    });
  };
  walk(mode, k, v, kt, lse, dot, rowscale, Lk, Lp);
  if (w2.k != nullptr) {
    __syncthreads();   // every wave is done with the first walk's stages
    walk(NSA_MODE_WINDOW, w2.k, w2.v, w2.kt, w2.lse, w2.dot, w2.rowscale, T_, w2.Lp);
  }

  if (sel_part != nullptr) {
    // finish the rows: dq_out = (dq if accumulate) + this branch's dQ + the
    // selection dQ partials of the row's valid slots (nsa_sel_dkdv's layout
    // [B][Hkv][T][NS][G][D]); the wave's tile goes through LDS so that every
    // partial is read as whole 16-byte row chunks
    static_assert(NT == 1, "one 32-row tile per wave is staged");
    __syncthreads();   // the key stages are free
    float* fin = reinterpret_cast<float*>(smem) + w * 32 * FIN_PITCH;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * h;
        if (D % 32 == 0 || d < D)
          *reinterpret_cast<f32x4*>(fin + n * FIN_PITCH + d) =
              (f32x4){acc[dt][0][4 * g4], acc[dt][0][4 * g4 + 1], acc[dt][0][4 * g4 + 2], acc[dt][0][4 * g4 + 3]} *
              scale;
      }
    __syncthreads();
    constexpr int CPR = D / 8, RPI = 64 / CPR;   // 8-element chunks per row, rows per pass
    const int c8 = lane % CPR, rsub = lane / CPR;
    const int nsub = sel_passes(sel_L), NS = S * nsub, n_csr = sel_csr_blocks(T_, sel_L);
    const int G = mp.G;
    for (int r0 = 0; r0 < 32; r0 += RPI) {
      const int r = r0 + rsub;
      int t, gl;   // query and head within the group
      range_row<FLAT>(rr, mp, 0, r, t, gl);
      if (t >= T_ || gl >= G) continue;
      const int64_t orow = ((int64_t)mp.b * Hq + mp.hkv * G + gl) * T_ + t;
      float v[8];
      {
        const f32x4 a = *reinterpret_cast<const f32x4*>(fin + r * FIN_PITCH + 8 * c8);
        const f32x4 b2 = *reinterpret_cast<const f32x4*>(fin + r * FIN_PITCH + 8 * c8 + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = a[i], v[4 + i] = b2[i];
      }
      if (accumulate) {
        float u[8];
        load8(dq + orow * D + 8 * c8, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += u[i];
      }
      const int64_t qrow_sel = (int64_t)bh * T_ + t;
      const int32_t* irow = sel_idx + qrow_sel * S;
      for (int s0 = 0; s0 < NS; s0 += 16) {
        Raw8<T> x[16];
        int jv[16];
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) {
          const int sl = s0 + k2 < NS ? s0 + k2 : NS - 1;
          jv[k2] = irow[sl / nsub];
          x[k2].load_nt(sel_part + ((qrow_sel * NS + sl) * G + gl) * D + 8 * c8);
        }
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) {
          x[k2].keep_if(s0 + k2 < NS && sel_slot_valid(jv[k2], n_csr, sel_L, t));
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] += x[k2].get(i);
        }
      }
      if (dq_out32 != nullptr)
        store8(dq_out32 + orow * D + 8 * c8, v);
      else
        store8_as<kWholeLines<D>>(dq_out + orow * D + 8 * c8, v);
    }
    return;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if (!rok[nt]) continue;
    float* qrow = dq + row[nt] * D;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * h;
        if (D % 32 == 0 || d < D) {
          f32x4 val = (f32x4){acc[dt][nt][4 * g4], acc[dt][nt][4 * g4 + 1], acc[dt][nt][4 * g4 + 2],
                              acc[dt][nt][4 * g4 + 3]} * scale;
          if (accumulate) val += *reinterpret_cast<const f32x4*>(qrow + d);
          *reinterpret_cast<f32x4*>(qrow + d) = val;
        }
      }
    }
  }
}

template <typename T> struct RangeNT { static constexpr int fwd = 1; static constexpr int dq = 1; };

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

static inline bool range_args_ok(int mode, int B, int Hq, int Hkv, int T, int Lk, int D, int window, int cl,
                                 int cd) {
  if (B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || T < 0 || Lk < 0) return false;
  if (!(D == 16 || D == 32 || D == 64 || D == 128)) return false;
  if (mode == NSA_MODE_WINDOW) return window >= 1 && Lk == T;
  return cl >= 1 && cd >= 1;
}

extern "C" {

}  // extern "C"

template <typename E, typename TO>
static int range_fwd_launch(int mode, const void* q, const void* k, const void* vt, void* o, float* lse, int B,
                            int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride,
                            const FwdExtras<E, TO>& fin, hipStream_t s) {
  const int NHC = (Hq / Hkv + 15) / 16;
  const int Lp = padded_len(Lk);
  const float sl2 = (1.0f / sqrtf((float)D)) * kLog2e;
  constexpr int NT = RangeNT<E>::fwd;
  const bool flat = Hq / Hkv < 16;   // flat rows: no empty head slots
  NSA_CHECK((int64_t)T * (Hq / Hkv) < (1ll << 31), NSA_ERR_SHAPE);
  const int nqt = range_qtiles(flat, T, Hq / Hkv, NT);
  const int64_t grid = (int64_t)B * Hkv * NHC * nqt;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  NSA_DISPATCH_D(D, {
    auto kern = flat ? k_range_fwd32<E, DD, NT, TO, true> : k_range_fwd32<E, DD, NT, TO, false>;
    kern<<<(unsigned)grid, 256, 0, s>>>(mode, (const E*)q, (const E*)k, (const E*)vt, (TO*)o, lse, Hq, Hkv, T, Lk,
                                        Lp, nqt, window, cmp_block, cmp_stride, sl2, fin);
  });
  return nsa_launch_status();
}

template <typename E>
static int range_dq_launch(int mode, const void* q, const void* k, const void* v, const void* kt, const void* dout,
                           const float* lse, const float* dot, const float* rowscale, float* dq, int accumulate,
                           int B, int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride,
                           const void* sel_part, const int32_t* sel_idx, int S, int sel_block, void* dq_out,
                           bool out_f32, const DqWindow<E>& w2, hipStream_t s) {
  const int NHC = (Hq / Hkv + 15) / 16;
  const int Lp = padded_len(Lk);
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  constexpr int NT = RangeNT<E>::dq;
  const bool flat = Hq / Hkv < 16;   // flat rows: no empty head slots
  NSA_CHECK((int64_t)T * (Hq / Hkv) < (1ll << 31), NSA_ERR_SHAPE);
  const int nqt = range_qtiles(flat, T, Hq / Hkv, NT);
  const int64_t grid = (int64_t)B * Hkv * NHC * nqt;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  NSA_DISPATCH_D(D, {
    auto kern = flat ? k_range_dq32<E, DD, NT, true> : k_range_dq32<E, DD, NT, false>;
    kern<<<(unsigned)grid, 256, 0, s>>>(mode, (const E*)q, (const E*)k, (const E*)v, (const E*)kt, (const E*)dout,
                                        lse, dot, rowscale, dq, accumulate, Hq, Hkv, T, Lk, Lp, nqt, window,
                                        cmp_block, cmp_stride, sl2, scale, (const E*)sel_part, sel_idx,
                                        out_f32 ? nullptr : (E*)dq_out, out_f32 ? (float*)dq_out : nullptr, S,
                                        sel_block, w2);
  });
  return nsa_launch_status();
}

extern "C" {

int nsa_range_fwd(int mode, const void* q, const void* k, const void* vt, void* o, float* lse, int B, int Hq,
                  int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride, void* q_packed, int dtype,
                  int o_dtype, void* stream) {
  NSA_CHECK(mode == NSA_MODE_WINDOW || mode == NSA_MODE_COMPRESS, NSA_ERR_ARG);
  NSA_CHECK(range_args_ok(mode, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(o_dtype == dtype || o_dtype == NSA_F32 || (o_dtype == NSA_F16S && dtype == NSA_BF16), NSA_ERR_DTYPE);
  if (T == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  NSA_CHECK(q_packed != q, NSA_ERR_ARG);
  if (o_dtype == NSA_F16S) {
    FwdExtras<bf16, f16> ex{};
    ex.q_packed = (bf16*)q_packed;
    ex.o_scale = f16s_scales(o, (int64_t)B * Hq * T, D);
    return range_fwd_launch<bf16, f16>(mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block,
                                       cmp_stride, ex, s);
  }
  if (dtype == NSA_BF16 && o_dtype == NSA_BF16) {
    FwdExtras<bf16, bf16> ex{};
    ex.q_packed = (bf16*)q_packed;
    return range_fwd_launch<bf16, bf16>(mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block,
                                        cmp_stride, ex, s);
  }
  if (dtype == NSA_BF16) {
    FwdExtras<bf16, float> ex{};
    ex.q_packed = (bf16*)q_packed;
    return range_fwd_launch<bf16, float>(mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block,
                                         cmp_stride, ex, s);
  }
  FwdExtras<float, float> ex{};
  ex.q_packed = (float*)q_packed;
  return range_fwd_launch<float, float>(mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block,
                                        cmp_stride, ex, s);
}

int nsa_range_fwd_finish(int mode, const void* q, const void* k, const void* vt, void* o, float* lse, int B,
                         int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride,
                         const void* o_part, const float* ml_part, const int32_t* block_idx, int S, int sel_block,
                         void* o_sel, float* lse_sel, const void* o_cmp, const void* gate, void* out, int dtype,
                         int o_dtype, int out_dtype, void* stream) {
  NSA_CHECK(mode == NSA_MODE_WINDOW || mode == NSA_MODE_COMPRESS, NSA_ERR_ARG);
  NSA_CHECK(range_args_ok(mode, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(o_dtype == dtype || o_dtype == NSA_F32 || (o_dtype == NSA_F16S && dtype == NSA_BF16), NSA_ERR_DTYPE);
  NSA_CHECK(o_part && ml_part && block_idx && o_sel && lse_sel && o_cmp && gate && out, NSA_ERR_ARG);
  NSA_CHECK(S >= 1 && sel_block >= 16 && sel_block % 16 == 0, NSA_ERR_SHAPE);
  NSA_CHECK(out_dtype == dtype || out_dtype == NSA_F32, NSA_ERR_DTYPE);
  if (T == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  float* out32 = out_dtype == NSA_F32 && dtype != NSA_F32 ? (float*)out : nullptr;
  if (out32 != nullptr) out = nullptr;
  if (o_dtype == NSA_F16S) {
    const int64_t rows = (int64_t)B * Hq * T;
    return range_fwd_launch<bf16, f16>(
        mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride,
        FwdExtras<bf16, f16>{nullptr, (const f16*)o_part, (const float2*)ml_part, block_idx, (f16*)o_sel,
                             lse_sel, (const f16*)o_cmp, (const bf16*)gate, (bf16*)out, S, sel_block, out32,
                             f16s_scales(o, rows, D), f16s_scales(o_sel, rows, D),
                             f16s_scales(const_cast<void*>(o_cmp), rows, D)},
        s);
  }
  if (dtype == NSA_BF16 && o_dtype == NSA_BF16)
    return range_fwd_launch<bf16, bf16>(
        mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride,
        FwdExtras<bf16, bf16>{nullptr, (const f16*)o_part, (const float2*)ml_part, block_idx, (bf16*)o_sel,
                              lse_sel, (const bf16*)o_cmp, (const bf16*)gate, (bf16*)out, S, sel_block,
                              out32},
        s);
  if (dtype == NSA_BF16)
    return range_fwd_launch<bf16, float>(
        mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride,
        FwdExtras<bf16, float>{nullptr, (const f16*)o_part, (const float2*)ml_part, block_idx, (float*)o_sel,
                               lse_sel, (const float*)o_cmp, (const bf16*)gate, (bf16*)out, S, sel_block,
                               out32},
        s);
  return range_fwd_launch<float, float>(
      mode, q, k, vt, o, lse, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride,
      FwdExtras<float, float>{nullptr, (const float*)o_part, (const float2*)ml_part, block_idx, (float*)o_sel,
                              lse_sel, (const float*)o_cmp, (const float*)gate, (float*)out, S, sel_block,
                              nullptr},
      s);
}

int nsa_range_dq(int mode, const void* q, const void* k, const void* v, const void* kt, const void* dout,
                 const float* lse, const float* dot, const float* rowscale, float* dq, int accumulate, int B,
                 int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride,
                 const void* sel_part, const int32_t* sel_idx, int S, int sel_block, void* dq_out, int dtype,
                 int dq_out_dtype, void* stream) {
  NSA_CHECK(mode == NSA_MODE_WINDOW || mode == NSA_MODE_COMPRESS, NSA_ERR_ARG);
  NSA_CHECK(dq_out_dtype == dtype || dq_out_dtype == NSA_F32, NSA_ERR_DTYPE);
  NSA_CHECK(range_args_ok(mode, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(sel_part == nullptr || (sel_idx != nullptr && dq_out != nullptr && S >= 1 && sel_block >= 16 &&
                                    sel_block % 16 == 0 && (!accumulate || dq != nullptr)),
            NSA_ERR_ARG);
  if (T == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NSA_BF16)
    return range_dq_launch<bf16>(mode, q, k, v, kt, dout, lse, dot, rowscale, dq, accumulate, B, Hq, Hkv, T, Lk,
                                 D, window, cmp_block, cmp_stride, sel_part, sel_idx, S, sel_block, dq_out,
                                 dq_out_dtype == NSA_F32, DqWindow<bf16>{}, s);
  return range_dq_launch<float>(mode, q, k, v, kt, dout, lse, dot, rowscale, dq, accumulate, B, Hq, Hkv, T, Lk, D,
                                window, cmp_block, cmp_stride, sel_part, sel_idx, S, sel_block, dq_out, false,
                                DqWindow<float>{}, s);
}

int nsa_range_dq_cw(const void* q, const void* dout, const void* kc, const void* vc, const void* ktc,
                    const float* lse_c, const float* dot_c, const float* rowscale_c, int Lk, int cmp_block,
                    int cmp_stride, const void* kw, const void* vw, const void* ktw, const float* lse_w,
                    const float* dot_w, const float* rowscale_w, int window, int B, int Hq, int Hkv, int T, int D,
                    const void* sel_part, const int32_t* sel_idx, int S, int sel_block, void* dq_out, int dtype,
                    int dq_out_dtype, void* stream) {
  NSA_CHECK(dq_out_dtype == dtype || dq_out_dtype == NSA_F32, NSA_ERR_DTYPE);
  NSA_CHECK(range_args_ok(NSA_MODE_COMPRESS, B, Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride) &&
                range_args_ok(NSA_MODE_WINDOW, B, Hq, Hkv, T, T, D, window, cmp_block, cmp_stride),
            NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(kw && vw && ktw && lse_w && dot_w && kc && vc && ktc && lse_c && dot_c && dq_out, NSA_ERR_ARG);
  NSA_CHECK(sel_part == nullptr || (sel_idx != nullptr && S >= 1 && sel_block >= 16 && sel_block % 16 == 0),
            NSA_ERR_ARG);
  NSA_CHECK(sel_part != nullptr, NSA_ERR_ARG);   // the rows are finished through the selection epilogue
  if (T == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int Lpw = padded_len(T);
  if (dtype == NSA_BF16)
    return range_dq_launch<bf16>(NSA_MODE_COMPRESS, q, kc, vc, ktc, dout, lse_c, dot_c, rowscale_c, nullptr, 0, B,
                                 Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride, sel_part, sel_idx, S, sel_block,
                                 dq_out, dq_out_dtype == NSA_F32,
                                 DqWindow<bf16>{(const bf16*)kw, (const bf16*)vw, (const bf16*)ktw, lse_w, dot_w,
                                                rowscale_w, Lpw},
                                 s);
  return range_dq_launch<float>(NSA_MODE_COMPRESS, q, kc, vc, ktc, dout, lse_c, dot_c, rowscale_c, nullptr, 0, B,
                                Hq, Hkv, T, Lk, D, window, cmp_block, cmp_stride, sel_part, sel_idx, S, sel_block,
                                dq_out, false,
                                DqWindow<float>{(const float*)kw, (const float*)vw, (const float*)ktw, lse_w, dot_w,
                                                rowscale_w, Lpw},
                                s);
}

}  // extern "C"
