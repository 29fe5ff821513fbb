// Query-side selection kernels: forward and dQ over the gathered blocks.
//
// One wave owns one 16-head column block of a query and streams its selected
// blocks in 32-key steps through nsa_tiles.h.  Workgroups are four waves over
// neighbouring queries of the same KV head, mapped onto one XCD so that
// shared blocks hit its L2.
#include "nsa_launch.h"
#include "nsa_tiles.h"

namespace nsa {

struct QueryMap {
  int b, hkv, hc, bh;
  int head0;   // first query head of the 16-head chunk
  int G, NHC;
};

__device__ __forceinline__ QueryMap map_bh_hc(int64_t r, int Hq, int Hkv) {
  QueryMap m;
  m.G = Hq / Hkv;
  m.NHC = (m.G + 15) / 16;
  m.hc = (int)(r % m.NHC);
  m.bh = (int)(r / m.NHC);
  m.b = m.bh / Hkv;
  m.hkv = m.bh % Hkv;
  m.head0 = m.hkv * m.G + m.hc * 16;
  return m;
}

// ---------------------------------------------------------------------------
// selection forward
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void k_sel_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                                 const T* __restrict__ vt, const int32_t* __restrict__ idx,
                                                 T* __restrict__ o, float* __restrict__ lse, int Hq, int Hkv,
                                                 int T_, int S, int L, int Lp, int nqb, float sl2) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const int64_t wg = xcd_remap(blockIdx.x, gridDim.x);
  const int t = (int)(wg % nqb) * 4 + w;
  const QueryMap m = map_bh_hc(wg / nqb, Hq, Hkv);
  if (t >= T_) return;
  const bool col_ok = m.hc * 16 + c < m.G;
  const int64_t row = ((int64_t)m.b * Hq + m.head0 + c) * T_ + t;
  Frag<T> qf[Dims<D>::KC];
  load_row_frags<T, D>(qf, col_ok ? q + row * D : nullptr, g);
  const T* kb_ = k + (int64_t)m.bh * T_ * D;
  const T* vtb = vt + (int64_t)m.bh * D * Lp;
  const int32_t* irow = idx + ((int64_t)m.bh * T_ + t) * S;
  FwdAcc<D> acc;
  acc.init();
  for (int s0 = 0; s0 < S; s0 += 64) {
    const int mine = s0 + lane < S ? irow[s0 + lane] : -1;
    const int ns = S - s0 < 64 ? S - s0 : 64;
    for (int s = 0; s < ns; ++s) {
      const int blk = __builtin_amdgcn_readlane(mine, s);
      if (blk < 0) continue;
      const int p0 = blk * L;
      if (p0 > t || p0 >= T_) continue;
      int pend = p0 + L < T_ ? p0 + L : T_;
      pend = pend < t + 1 ? pend : t + 1;
      for (int kb = p0; kb < pend; kb += 32) {
        Frag<T> kf[2][Dims<D>::KC];
        Frag<T> vf[Dims<D>::DT];
        load_key_frags<T, D>(kf, kb_, kb, pend, g, c);
        load_t_frags<T, D>(vf, vtb, Lp, kb, g, c);
        const uint32_t vm = col_ok ? range_mask(kb + 8 * g, p0, pend - 1) : 0u;
        fwd_step<T, D>(acc, qf, kf, vf, vm, sl2);
      }
    }
  }
  fwd_store<T, D>(acc, col_ok ? o + row * D : nullptr, lse + row, g);
}

// ---------------------------------------------------------------------------
// dQ kernels
// ---------------------------------------------------------------------------
struct DqRow {
  float lse2, rs, dot;
};

__device__ __forceinline__ DqRow load_dq_row(const float* lse, const float* rowscale, const float* dot,
                                             int64_t r, bool ok) {
  DqRow d;
  d.lse2 = ok ? lse[r] * kLog2e : 0.0f;
  d.rs = (ok && rowscale != nullptr) ? rowscale[r] : 1.0f;
  d.dot = ok ? dot[r] : 0.0f;
  return d;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void k_sel_dq(const T* __restrict__ q, const T* __restrict__ k,
                                                const T* __restrict__ v, const T* __restrict__ kt,
                                                const T* __restrict__ dout, const int32_t* __restrict__ idx,
                                                const float* __restrict__ lse, const float* __restrict__ dot,
                                                const float* __restrict__ rowscale, float* __restrict__ dq,
                                                int accumulate, int Hq, int Hkv, int T_, int S, int L, int Lp,
                                                int nqb, float sl2, float scale) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const int64_t wg = xcd_remap(blockIdx.x, gridDim.x);
  const int t = (int)(wg % nqb) * 4 + w;
  const QueryMap m = map_bh_hc(wg / nqb, Hq, Hkv);
  if (t >= T_) return;
  const bool col_ok = m.hc * 16 + c < m.G;
  const int64_t row = ((int64_t)m.b * Hq + m.head0 + c) * T_ + t;
  Frag<T> qf[Dims<D>::KC], df[Dims<D>::KC];
  load_row_frags<T, D>(qf, col_ok ? q + row * D : nullptr, g);
  load_row_frags<T, D>(df, col_ok ? dout + row * D : nullptr, g);
  const DqRow rs = load_dq_row(lse, rowscale, dot, row, col_ok);
  const T* kb_ = k + (int64_t)m.bh * T_ * D;
  const T* vb_ = v + (int64_t)m.bh * T_ * D;
  const T* ktb = kt + (int64_t)m.bh * D * Lp;
  const int32_t* irow = idx + ((int64_t)m.bh * T_ + t) * S;
  f32x4 acc[Dims<D>::DT];
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) acc[dt] = zero4();
  for (int s0 = 0; s0 < S; s0 += 64) {
    const int mine = s0 + lane < S ? irow[s0 + lane] : -1;
    const int ns = S - s0 < 64 ? S - s0 : 64;
    for (int s = 0; s < ns; ++s) {
      const int blk = __builtin_amdgcn_readlane(mine, s);
      if (blk < 0) continue;
      const int p0 = blk * L;
      if (p0 > t || p0 >= T_) continue;
      int pend = p0 + L < T_ ? p0 + L : T_;
      pend = pend < t + 1 ? pend : t + 1;
      for (int kb = p0; kb < pend; kb += 32) {
        Frag<T> kf[2][Dims<D>::KC], vf[2][Dims<D>::KC];
        Frag<T> ktf[Dims<D>::DT];
        load_key_frags<T, D>(kf, kb_, kb, pend, g, c);
        load_key_frags<T, D>(vf, vb_, kb, pend, g, c);
        load_t_frags<T, D>(ktf, ktb, Lp, kb, g, c);
        const uint32_t vm = col_ok ? range_mask(kb + 8 * g, p0, pend - 1) : 0u;
        dq_step<T, D>(acc, qf, df, kf, vf, ktf, vm, sl2, rs.lse2, rs.rs, rs.dot);
      }
    }
  }
  if (col_ok) dq_store<D>(acc, dq + row * D, g, scale, accumulate != 0);
}

// ---------------------------------------------------------------------------
// dispatch helpers
// ---------------------------------------------------------------------------
#define NSA_DISPATCH_D(D_, ...)                  \
  switch (D_) {                                  \
    case 16: { constexpr int DD = 16; __VA_ARGS__; break; } \
    case 32: { constexpr int DD = 32; __VA_ARGS__; break; } \
    case 64: { constexpr int DD = 64; __VA_ARGS__; break; } \
    case 128: { constexpr int DD = 128; __VA_ARGS__; break; } \
    default: return NSA_ERR_SHAPE;               \
  }

}  // namespace nsa

using namespace nsa;

static inline bool nsa_dtype_ok(int dtype) { return dtype == NSA_F32 || dtype == NSA_BF16; }
static inline bool nsa_d_ok(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }

extern "C" {

int nsa_version(void) { return 100; }

int nsa_padded_len(int Lk) { return nsa::padded_len(Lk); }

int nsa_sel_fwd(const void* q, const void* k, const void* vt, const int32_t* block_idx, void* o, float* lse,
                int B, int Hq, int Hkv, int T, int D, int S, int block_size, int dtype, void* stream) {
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && S >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(nsa_d_ok(D) && block_size >= 16 && block_size % 16 == 0, NSA_ERR_SHAPE);
  NSA_CHECK(nsa_dtype_ok(dtype), NSA_ERR_DTYPE);
  if (T == 0) return NSA_OK;
  const int G = Hq / Hkv, NHC = (G + 15) / 16, nqb = (T + 3) / 4;
  const int64_t grid = (int64_t)B * Hkv * NHC * nqb;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  const int Lp = nsa::padded_len(T);
  const float sl2 = (1.0f / sqrtf((float)D)) * nsa::kLog2e;
  hipStream_t s = (hipStream_t)stream;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16)
      k_sel_fwd<bf16, DD><<<(unsigned)grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)vt,
                                                         block_idx, (bf16*)o, lse, Hq, Hkv, T, S, block_size, Lp,
                                                         nqb, sl2);
    else
      k_sel_fwd<float, DD><<<(unsigned)grid, 256, 0, s>>>((const float*)q, (const float*)k, (const float*)vt,
                                                          block_idx, (float*)o, lse, Hq, Hkv, T, S, block_size,
                                                          Lp, nqb, sl2);
  });
  return nsa_launch_status();
}

int nsa_sel_dq(const void* q, const void* k, const void* v, const void* kt, const void* dout,
               const int32_t* block_idx, const float* lse, const float* dot, const float* rowscale, float* dq,
               int accumulate, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int dtype,
               void* stream) {
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && S >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(nsa_d_ok(D) && block_size >= 16 && block_size % 16 == 0, NSA_ERR_SHAPE);
  NSA_CHECK(nsa_dtype_ok(dtype), NSA_ERR_DTYPE);
  if (T == 0) return NSA_OK;
  const int G = Hq / Hkv, NHC = (G + 15) / 16, nqb = (T + 3) / 4;
  const int64_t grid = (int64_t)B * Hkv * NHC * nqb;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  const int Lp = nsa::padded_len(T);
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * nsa::kLog2e;
  hipStream_t s = (hipStream_t)stream;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16)
      k_sel_dq<bf16, DD><<<(unsigned)grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v,
                                                        (const bf16*)kt, (const bf16*)dout, block_idx, lse, dot,
                                                        rowscale, dq, accumulate, Hq, Hkv, T, S, block_size, Lp,
                                                        nqb, sl2, scale);
    else
      k_sel_dq<float, DD><<<(unsigned)grid, 256, 0, s>>>((const float*)q, (const float*)k, (const float*)v,
                                                         (const float*)kt, (const float*)dout, block_idx, lse,
                                                         dot, rowscale, dq, accumulate, Hq, Hkv, T, S,
                                                         block_size, Lp, nqb, sl2, scale);
  });
  return nsa_launch_status();
}

}  // extern "C"
