// Block importance + top-n selection (the block choice of NSAAttention,
// nsa_model.py:245-258 and :343-355), one wave per (b, hkv, t).
//
//  1. p_cmp = exp2(q.k_cmp * scale*log2e - lse_cmp*log2e) over the visible
//     pooled tokens (lse_cmp from the compression forward), 32 tokens per MFMA
//     step, summed over the 16 heads of each head chunk with a butterfly
//     inside the 16-lane groups, accumulated per token in LDS (head chunks in
//     order, so the sum order is fixed).
//  2. imp_slc[j] = sum_i imp_cmp[i] * |span_i & block_j| / d (tokens ascending).
//  3. score = +inf for forced blocks, -FLT_MAX for blocks not yet complete,
//     else imp_slc; keys (orderable score << 32 | ~j) make a wave-wide u64 max
//     pick the highest score and, among equal scores, the lowest block index.
#include "nsa_launch.h"
#include "nsa_tiles.h"

namespace nsa {

__device__ __forceinline__ uint64_t topn_key(float x, int j) {
  uint32_t u = __float_as_uint(x);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)j);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((unsigned)(v & 0xFFFFFFFFu), m, kWave);
  const uint32_t hi = __shfl_xor((unsigned)(v >> 32), m, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ void wave_fence() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

template <typename T, int D>
__global__ __launch_bounds__(256) void k_topn(const T* __restrict__ q, const T* __restrict__ kc,
                                              const float* __restrict__ lse, int32_t* __restrict__ out_idx,
                                              float* __restrict__ scores, int Hq, int Hkv, int T_, int n_cmp,
                                              int ncp, int n_slc, int S, int cl, int cd, int ls, int force_init,
                                              int n_local, int wpb, int64_t nrows, float sl2) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const int64_t r = (int64_t)blockIdx.x * wpb + w;
  if (r >= nrows) return;
  float* imp = smem + (int64_t)w * (ncp + n_slc);
  float* sc = imp + ncp;
  const int t = (int)(r % T_);
  const int bh = (int)(r / T_);
  const int b = bh / Hkv, hkv = bh % Hkv;
  const int G = Hq / Hkv, NHC = (G + 15) / 16;
  for (int i = lane; i < ncp; i += kWave) imp[i] = 0.0f;
  wave_fence();

  int hi = -1;
  if (t >= cl - 1 && n_cmp > 0) {
    hi = (t - cl + 1) / cd;
    hi = hi < n_cmp - 1 ? hi : n_cmp - 1;
  }
  const T* kbase = kc + (int64_t)bh * n_cmp * D;
  for (int hc = 0; hc < NHC; ++hc) {
    const int hg = hc * 16 + c;
    const bool col_ok = hg < G;
    const int64_t row = ((int64_t)b * Hq + hkv * G + hg) * T_ + t;
    Frag<T> qf[Dims<D>::KC];
    load_row_frags<T, D>(qf, col_ok ? q + row * D : nullptr, g);
    const float lse2 = col_ok ? lse[row] * kLog2e : 0.0f;
    for (int kb = 0; kb <= hi; kb += 32) {
      Frag<T> kf[2][Dims<D>::KC];
      load_key_frags<T, D>(kf, kbase, kb, n_cmp, g, c);
      f32x4 s0 = zero4(), s1 = zero4();
#pragma unroll
      for (int kc2 = 0; kc2 < Dims<D>::KC; ++kc2) {
        mma(s0, kf[0][kc2], qf[kc2]);
        mma(s1, kf[1][kc2], qf[kc2]);
      }
      const uint32_t vm = col_ok ? range_mask(kb + 8 * g, 0, hi) : 0u;
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float s = j < 4 ? s0[j & 3] : s1[j & 3];
        p[j] = ((vm >> j) & 1u) ? fast_exp2(s * sl2 - lse2) : 0.0f;
      }
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] += __shfl_xor(p[j], m, kWave);
      }
      float mine = p[0];
#pragma unroll
      for (int j = 1; j < 8; ++j) mine = (c == j) ? p[j] : mine;
      const int tok = kb + 8 * g + c;
      if (c < 8 && tok < ncp) imp[tok] += mine;
    }
    wave_fence();
  }

  // selection-block importance, masking and forcing
  const int tb = t / ls;
  for (int j = lane; j < n_slc; j += kWave) {
    const int lo_i = j * ls - cl + 1 <= 0 ? 0 : (j * ls - cl + 1 + cd - 1) / cd;
    int hi_i = ((j + 1) * ls - 1) / cd;
    hi_i = hi_i < n_cmp - 1 ? hi_i : n_cmp - 1;
    float s = 0.0f;
    for (int i = lo_i; i <= hi_i; ++i) {
      const int a = i * cd > j * ls ? i * cd : j * ls;
      const int e = i * cd + cl < (j + 1) * ls ? i * cd + cl : (j + 1) * ls;
      if (e > a) s += imp[i] * ((float)(e - a) / (float)cd);
    }
    if (scores != nullptr) scores[r * n_slc + j] = s;
    const bool valid = (j + 1) * ls - 1 <= t;
    const bool forced = (force_init && j == 0) || (j <= tb && j > tb - n_local);
    sc[j] = forced ? __builtin_inff() : (valid ? s : -3.4028234663852886e38f);
  }
  wave_fence();

  // top-S: wave-wide argmax of (score, lower index), S times
  uint64_t removed = 0;
  auto lane_best = [&]() {
    uint64_t best = 0;
    int k = 0;
    for (int j = lane; j < n_slc; j += kWave, ++k) {
      if ((removed >> k) & 1ull) continue;
      const uint64_t key = topn_key(sc[j], j);
      best = key > best ? key : best;
    }
    return best;
  };
  uint64_t mine = lane_best();
  int32_t* orow = out_idx + r * S;
  for (int s = 0; s < S; ++s) {
    uint64_t bk = mine;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const uint64_t o = shfl_xor_u64(bk, m);
      bk = o > bk ? o : bk;
    }
    const int jw = (int)(0xFFFFFFFFu - (uint32_t)(bk & 0xFFFFFFFFu));
    if (lane == 0) orow[s] = jw;
    if ((jw & (kWave - 1)) == lane) {
      removed |= 1ull << (jw / kWave);
      mine = lane_best();
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
  const int ncp = ((n_cmp + 31) / 32) * 32 + 32;
  const size_t per_wave = (size_t)(ncp + n_slc) * sizeof(float);
  NSA_CHECK(per_wave <= 65536, NSA_ERR_SHAPE);
  int wpb = (int)(65536 / per_wave);
  wpb = wpb > 4 ? 4 : wpb;
  const int64_t nrows = (int64_t)B * Hkv * T;
  const int64_t grid = (nrows + wpb - 1) / wpb;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  const float sl2 = (1.0f / sqrtf((float)D)) * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  const size_t lds = per_wave * wpb;
  switch (D) {
#define NSA_TOPN_CASE(DD)                                                                                        \
  case DD:                                                                                                       \
    if (dtype == NSA_BF16)                                                                                       \
      k_topn<bf16, DD><<<(unsigned)grid, 64 * wpb, lds, s>>>((const bf16*)q, (const bf16*)k_cmp, lse_cmp,      \
                                                             block_idx, scores, Hq, Hkv, T, n_cmp, ncp, n_slc, S, \
                                                             cmp_block, cmp_stride, sel_block, force_init,       \
                                                             n_local, wpb, nrows, sl2);                          \
    else                                                                                                         \
      k_topn<float, DD><<<(unsigned)grid, 64 * wpb, lds, s>>>((const float*)q, (const float*)k_cmp, lse_cmp,   \
                                                              block_idx, scores, Hq, Hkv, T, n_cmp, ncp, n_slc,  \
                                                              S, cmp_block, cmp_stride, sel_block, force_init,   \
                                                              n_local, wpb, nrows, sl2);                         \
    break;
    NSA_TOPN_CASE(16)
    NSA_TOPN_CASE(32)
    NSA_TOPN_CASE(64)
    NSA_TOPN_CASE(128)
#undef NSA_TOPN_CASE
    default:
      return NSA_ERR_SHAPE;
  }
  return nsa_launch_status();
}

}  // extern "C"
