// Wave-level attention tiles shared by the forward, dQ and dK/dV kernels.
//
// Query-side selection kernels (forward, dQ) and the importance kernel work on
// one query x 16 heads per N-tile and 32 keys per step:
//   S^T (32 keys x 16 heads) = K Q^T      two 16x16 accumulators
//   O^T (D x 16 heads)     += V^T P^T    D/16 accumulators
//   dQ^T (D x 16 heads)    += K^T dS^T
#pragma once

#include "nsa_common.h"

namespace nsa {

template <int D> struct Dims {
  static constexpr int KC = (D + 31) / 32;   // 32-wide K chunks over D
  static constexpr int DT = D / 16;          // 16-row tiles over D
};

// bits j (0..7) with lo <= base + j <= hi
__device__ __forceinline__ uint32_t range_mask(int base, int lo, int hi) {
  const int a = lo - base > 0 ? lo - base : 0;
  const int b = hi - base < 7 ? hi - base : 7;
  if (b < a) return 0u;
  return ((1u << (b + 1)) - 1u) & ~((1u << a) - 1u);
}

// Row fragments of a [.][D] row-major matrix as B operand of S^T (or A operand
// of S): lane (g, c) holds row `row` (the lane's head), d = 32*kc + 8g .. +7.
template <typename T, int D>
__device__ __forceinline__ void load_row_frags(Frag<T> (&f)[Dims<D>::KC], const T* row, int g) {
#pragma unroll
  for (int kc = 0; kc < Dims<D>::KC; ++kc) {
    if (row != nullptr && 32 * kc + 8 * g < D)
      f[kc].load(row + 32 * kc + 8 * g);
    else
      f[kc].zero();
  }
}

// Key rows of a 32-key step as the A operand of S^T = K Q^T (or of
// dP^T = V dO^T).  Row m = c of tile mt reads key kb + 8(c>>2) + 4mt + (c&3),
// which puts keys kb + 8g .. kb + 8g + 7 into lane group g of the C layout.
template <typename T, int D>
__device__ __forceinline__ void load_key_frags(Frag<T> (&f)[2][Dims<D>::KC], const T* base, int kb, int kend,
                                               int g, int c) {
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int key = kb + 8 * (c >> 2) + 4 * mt + (c & 3);
    const bool ok = key >= 0 && key < kend;
#pragma unroll
    for (int kc = 0; kc < Dims<D>::KC; ++kc) {
      if (ok && 32 * kc + 8 * g < D)
        f[mt][kc].load(base + (int64_t)key * D + 32 * kc + 8 * g);
      else
        f[mt][kc].zero();
    }
  }
}

// Transposed-copy fragments (A operand of O^T += V^T P^T / dQ^T += K^T dS^T):
// lane (g, c) reads row d = 16 dt + c, keys kb + 8g .. kb + 8g + 7.
template <typename T, int D>
__device__ __forceinline__ void load_t_frags(Frag<T> (&f)[Dims<D>::DT], const T* tbase, int Lp, int kb, int g,
                                             int c) {
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) f[dt].load(tbase + (int64_t)(16 * dt + c) * Lp + kb + 8 * g);
}

// ---------------------------------------------------------------------------
// forward online-softmax state of one 16-column query tile
// ---------------------------------------------------------------------------
template <int D> struct FwdAcc {
  float m;                  // running max of scaled scores (log2 units), equal on the 4 lane groups
  float l;                  // this lane's partial denominator
  f32x4 o[Dims<D>::DT];     // O^T: lane (g, c) holds rows d = 16dt + 4g + i of column c
  __device__ __forceinline__ void init() {
    m = kMaskScore;
    l = 0.0f;
#pragma unroll
    for (int dt = 0; dt < Dims<D>::DT; ++dt) o[dt] = zero4();
  }
};

template <typename T, int D>
__device__ __forceinline__ void fwd_step(FwdAcc<D>& a, const Frag<T> (&qf)[Dims<D>::KC],
                                         const Frag<T> (&kf)[2][Dims<D>::KC], const Frag<T> (&vf)[Dims<D>::DT],
                                         uint32_t vm, float sl2) {
  f32x4 s0 = zero4(), s1 = zero4();
#pragma unroll
  for (int kc = 0; kc < Dims<D>::KC; ++kc) {
    mma(s0, kf[0][kc], qf[kc]);
    mma(s1, kf[1][kc], qf[kc]);
  }
  float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  float mx = kMaskScore;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sv[j] = ((vm >> j) & 1u) ? sv[j] * sl2 : kMaskScore;
    mx = fmaxf(mx, sv[j]);
  }
  mx = group4_max(mx);
  const float mn = fmaxf(a.m, mx);
  const float alpha = fast_exp2(a.m - mn);
  float p[8];
  float ps = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    p[j] = ((vm >> j) & 1u) ? fast_exp2(sv[j] - mn) : 0.0f;
    ps += p[j];
  }
  a.l = a.l * alpha + ps;
  a.m = mn;
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) a.o[dt] *= alpha;
  Frag<T> pf;
  pf.set(p);
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) mma(a.o[dt], vf[dt], pf);
}

// Normalise and store one query tile: o[.. + 16dt + 4g + i] and lse (g == 0).
template <typename T, int D>
__device__ __forceinline__ void fwd_store(const FwdAcc<D>& a, T* orow, float* lse_ptr, int g) {
  const float lt = group4_sum(a.l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (orow != nullptr) {
#pragma unroll
    for (int dt = 0; dt < Dims<D>::DT; ++dt)
      store4(orow + 16 * dt + 4 * g, a.o[dt][0] * inv, a.o[dt][1] * inv, a.o[dt][2] * inv, a.o[dt][3] * inv);
    if (g == 0) *lse_ptr = lt > 0.0f ? (a.m + __log2f(lt)) * kLn2 : kLseEmpty;
  }
}

// ---------------------------------------------------------------------------
// dQ step of one 16-column query tile over 32 keys
// ---------------------------------------------------------------------------
template <typename T, int D>
__device__ __forceinline__ void dq_step(f32x4 (&dq)[Dims<D>::DT], const Frag<T> (&qf)[Dims<D>::KC],
                                        const Frag<T> (&df)[Dims<D>::KC], const Frag<T> (&kf)[2][Dims<D>::KC],
                                        const Frag<T> (&vf)[2][Dims<D>::KC], const Frag<T> (&ktf)[Dims<D>::DT],
                                        uint32_t vm, float sl2, float lse2, float rs, float dot) {
  f32x4 s0 = zero4(), s1 = zero4(), p0 = zero4(), p1 = zero4();
#pragma unroll
  for (int kc = 0; kc < Dims<D>::KC; ++kc) {
    mma(s0, kf[0][kc], qf[kc]);
    mma(s1, kf[1][kc], qf[kc]);
    mma(p0, vf[0][kc], df[kc]);
    mma(p1, vf[1][kc], df[kc]);
  }
  float ds[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float s = j < 4 ? s0[j & 3] : s1[j & 3];
    const float dp = j < 4 ? p0[j & 3] : p1[j & 3];
    const float p = ((vm >> j) & 1u) ? fast_exp2(s * sl2 - lse2) * rs : 0.0f;
    ds[j] = p * (dp - dot);
  }
  Frag<T> dsf;
  dsf.set(ds);
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) mma(dq[dt], ktf[dt], dsf);
}

template <int D>
__device__ __forceinline__ void dq_store(const f32x4 (&dq)[Dims<D>::DT], float* row, int g, float scale,
                                         bool accumulate) {
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) {
    float* p = row + 16 * dt + 4 * g;
    f32x4 v = dq[dt] * scale;
    if (accumulate) v += *reinterpret_cast<const f32x4*>(p);
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

}  // namespace nsa
