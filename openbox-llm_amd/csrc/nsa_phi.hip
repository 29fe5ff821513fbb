// Compression phi of the NSA paper (arXiv:2502.11089, eq. 7): the pooled
// token of span i is phi(x[i d .. i d + l - 1] + P) with a learnable MLP over
// the l x D span and an intra-block position encoding P (l x D):
//
//   pre_i = W1 vec(x_span_i + P) + b1 = W1 vec(x_span_i) + c1,  c1 = W1 vec(P) + b1
//   out_i = W2 silu(pre_i) + b2                 (W1: H x lD, W2: D x H)
//
// It replaces the reference's weighted mean + linear (BlockCompressor,
// nsa_model.py:100-123).  The span rows are contiguous in a [T][D] sequence,
// so span i is the lD-element row starting at x + i d D: the kernels read the
// overlapping spans in place (no unfolded copy).
//
// k_phi_fwd: one workgroup of four waves per 32 pooled tokens.  pre^T = W1
// X^T on 32x32x16 MFMAs with the hidden units on M (W1 rows, perm32 order)
// and the tokens on N; the waves split the lD contraction in quarters (one
// wave alone, streaming W1 and the spans from memory, is bound by the
// latency of its loads).  The quarters meet in LDS and are summed in wave
// order; wave mt then holds hidden tile mt, whose registers 8u .. 8u+7 of lane
// half h are hidden units 32 mt + 16 u + 8 h + j: after bias and SiLU they are
// the B operand of out^T = W2 silu(pre)^T for contraction step 2 mt + u, handed
// to the other waves through LDS in that same lane layout.  Wave dt computes
// output tile dt.  pre is kept (float) for the backward.
// k_phi_dpre: dpre = (W2^T dout) * silu'(pre), the same orientation.
// k_phi_fold: dx[p] = sum over the spans i that hold p of dspan_i[p - i d]
// (deterministic gather, no atomics).
// k_phi_wgrad / k_phi_wgrad_reduce: the parameter gradients (below).
#include "nsa_launch.h"
#include "nsa_tile32.h"

namespace nsa {

__device__ __forceinline__ float silu_f(float z) { return z / (1.0f + __expf(-z)); }
__device__ __forceinline__ float silu_grad(float z) {
  const float s = 1.0f / (1.0f + __expf(-z));
  return s * (1.0f + z * (1.0f - s));
}

// 8 consecutive elements starting at an 8-aligned index of a row of T
template <typename T>
__device__ __forceinline__ void store_run8(T* p, const float* v) {
  Frag<T> f;
  f.set(v);
  f.store(p);
}

constexpr int kPhiFwdWaves = 4;   // waves per 32 pooled tokens, each a quarter of the contraction

template <typename T, int D, int H>
__global__ __launch_bounds__(64 * kPhiFwdWaves) void k_phi_fwd(const T* __restrict__ x, const T* __restrict__ w1,
                                                               const float* __restrict__ c1,
                                                               const T* __restrict__ w2, const float* __restrict__ b2,
                                                               T* __restrict__ out, float* __restrict__ pre_out,
                                                               int BH, int L, int n, int l, int d, int ntile) {
  constexpr int NW = kPhiFwdWaves;
  constexpr int MT = H / 32;   // hidden tiles
  constexpr int DT = D / 32;   // output tiles
  static_assert(MT <= NW && DT <= NW, "one hidden / output tile per wave");
  __shared__ float part[NW][MT][16][64];              // each wave's partial pre^T, [register][lane]
  __shared__ __align__(16) T hbs[MT][2][64 * 8];      // silu(pre)^T B fragments, [lane][8]
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, nn = lane & 31;
  const int64_t wt = blockIdx.x;
  if (wt >= (int64_t)BH * ntile) return;   // uniform over the workgroup
  const int bh = (int)(wt / ntile), i0 = (int)(wt % ntile) * 32;
  const int K = l * D, KW = K / NW;        // D >= 64: KW is a multiple of 16
  const int tok = i0 + nn;
  const bool tok_ok = tok < n;
  // the B operand: token column nn reads its span row (tokens past n repeat the last)
  const T* xrow = x + ((int64_t)bh * L + (int64_t)(tok_ok ? tok : n - 1) * d) * D + 8 * h;
  const T* w1row[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) w1row[mt] = w1 + (int64_t)(32 * mt + perm32(nn)) * K + 8 * h;
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = zero16();
#pragma unroll 4
  for (int k0 = w * KW; k0 < (w + 1) * KW; k0 += 16) {
    Frag<T> bx;
    bx.load(xrow + k0);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      Frag<T> aw;
      aw.load(w1row[mt] + k0);
      mma32(acc[mt], aw, bx);
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) part[w][mt][r][lane] = acc[mt][r];
  __syncthreads();
  // wave mt: the quarters of hidden tile mt summed in wave order, bias, keep
  // pre, SiLU -> B fragments of silu(pre)^T
  if (w < MT) {
    const int mt = w;
    float pv[16], hv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float a = part[0][mt][r][lane];
#pragma unroll
      for (int q = 1; q < NW; ++q) a += part[q][mt][r][lane];
      pv[r] = a + c1[32 * mt + acc_elem(h, r)];
      hv[r] = silu_f(pv[r]);
    }
    if (tok_ok) {
      float* prow = pre_out + ((int64_t)bh * n + tok) * H;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float* p = prow + 32 * mt + 16 * u + 8 * h;
        *reinterpret_cast<f32x4*>(p) = (f32x4){pv[8 * u], pv[8 * u + 1], pv[8 * u + 2], pv[8 * u + 3]};
        *reinterpret_cast<f32x4*>(p + 4) = (f32x4){pv[8 * u + 4], pv[8 * u + 5], pv[8 * u + 6], pv[8 * u + 7]};
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      Frag<T> f;
      f.set(hv + 8 * u);
      f.store(&hbs[mt][u][lane * 8]);
    }
  }
  __syncthreads();
  // wave dt: out^T tile dt = W2 silu(pre)^T (A = W2 rows in perm32 order,
  // contraction over the hidden units)
  if (w < DT) {
    const int dt = w;
    f32x16 o = zero16();
    const T* w2row = w2 + (int64_t)(32 * dt + perm32(nn)) * H + 8 * h;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        Frag<T> a, hb;
        a.load(w2row + 32 * mt + 16 * u);
        hb.load(&hbs[mt][u][lane * 8]);
        mma32(o, a, hb);
      }
    if (tok_ok) {
      T* orow = out + ((int64_t)bh * n + tok) * D;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int d0 = 32 * dt + 16 * u + 8 * h;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = o[8 * u + j] + b2[d0 + j];
        store_run8(orow + d0, v);
      }
    }
  }
}

// dpre = (W2^T dout) * silu'(pre): w2t is W2^T [H][D]; dout [BH][n][D]; dpre float [BH][n][H]
template <typename T, int D, int H>
__global__ __launch_bounds__(256) void k_phi_dpre(const T* __restrict__ dout, const T* __restrict__ w2t,
                                                  const float* __restrict__ pre, float* __restrict__ dpre, int BH,
                                                  int n, int ntile) {
  constexpr int MT = H / 32, KS = D / 16;
  const int lane = threadIdx.x & 63, h = lane >> 5, nn = lane & 31;
  const int64_t wt = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wt >= (int64_t)BH * ntile) return;
  const int bh = (int)(wt / ntile), i0 = (int)(wt % ntile) * 32;
  const int tok = i0 + nn;
  const bool tok_ok = tok < n;
  const T* drow = dout + ((int64_t)bh * n + (tok_ok ? tok : n - 1)) * D + 8 * h;
  Frag<T> bd[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) bd[s].load(drow + 16 * s);
  const int64_t r0 = ((int64_t)bh * n + tok) * H;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x16 acc = zero16();
    const T* arow = w2t + (int64_t)(32 * mt + perm32(nn)) * D + 8 * h;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      Frag<T> a;
      a.load(arow + 16 * s);
      mma32(acc, a, bd[s]);
    }
    if (tok_ok) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int64_t o = r0 + 32 * mt + 16 * u + 8 * h;
        const f32x4 z0 = *reinterpret_cast<const f32x4*>(pre + o);
        const f32x4 z1 = *reinterpret_cast<const f32x4*>(pre + o + 4);
        f32x4 g0, g1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          g0[j] = acc[8 * u + j] * silu_grad(z0[j]);
          g1[j] = acc[8 * u + 4 + j] * silu_grad(z1[j]);
        }
        *reinterpret_cast<f32x4*>(dpre + o) = g0;
        *reinterpret_cast<f32x4*>(dpre + o + 4) = g1;
      }
    }
  }
}

// dx[bh][p][c] = sum over spans i with i d <= p < i d + l (i < n) of
// dspan[bh][i][(p - i d) D + c], spans ascending
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_phi_fold(const TI* __restrict__ dspan, TO* __restrict__ dx, int BH,
                                                  int L, int D, int n, int l, int d) {
  const int64_t total = (int64_t)BH * L * D;
  const int64_t K = (int64_t)l * D;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % D);
    const int64_t r = e / D;
    const int p = (int)(r % L);
    const int64_t bh = r / L;
    int ilo = p - l + 1 <= 0 ? 0 : (p - l + 1 + d - 1) / d;
    int ihi = p / d;
    ihi = ihi < n - 1 ? ihi : n - 1;
    float s = 0.0f;
    for (int i = ilo; i <= ihi; ++i) s += to_f32(dspan[(bh * n + i) * K + (int64_t)(p - i * d) * D + c]);
    dx[e] = from_f32<TO>(s);
  }
}

// k_phi_fold for D a multiple of 8: a thread sums 8 consecutive channels of
// one position (16-byte loads of 16-bit data), spans ascending as above, so
// the sums are the same bits
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_phi_fold8(const TI* __restrict__ dspan, TO* __restrict__ dx, int BH,
                                                   int L, int D, int n, int l, int d) {
  const int C8 = D / 8;
  const int64_t total = (int64_t)BH * L * C8;
  const int64_t K = (int64_t)l * D;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % C8) * 8;
    const int64_t r = e / C8;
    const int p = (int)(r % L);
    const int64_t bh = r / L;
    int ilo = p - l + 1 <= 0 ? 0 : (p - l + 1 + d - 1) / d;
    int ihi = p / d;
    ihi = ihi < n - 1 ? ihi : n - 1;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i = ilo; i <= ihi; ++i) {
      float v[8];
      load8(dspan + (bh * n + i) * K + (int64_t)(p - i * d) * D + c, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] += v[j];
    }
    store8(dx + r * D + c, s);
  }
}

// Weight gradients of phi, over the M = BH n pooled tokens g:
//   dW1[u][k] = sum_g dpre[g][u] vec(span_g)[k] + db1[u] vec(P)[k]
//   dW2[c][u] = sum_g dout[g][c] silu(pre[g][u])
//   db1[u] = sum_g dpre[g][u],  db2[c] = sum_g dout[g][c],  dpos = db1^T W1 as [l][D]
// k_phi_wgrad contracts over the tokens on 32x32x16 MFMAs, hidden units on M:
// a workgroup owns 128 output columns (wave w: columns 32 w .. 32 w + 31 of
// every hidden tile) of W1's span columns (groups 0 .. ncg1 - 1) or of dW2^T
// (group ncg1, dout's channels), and one of `nsplit` token ranges (grid.y),
// whose sums it writes as float partials.  Both operands are token-major in
// memory; each 32-token chunk is staged in LDS transposed, token-contiguous
// rows of which a lane reads 8.  Span g's element k is x[bh][(i d) D + k]
// (rows i d .. i d + l - 1 are contiguous): the spans are read in place.  bf16:
// dpre / silu(pre) enter as bf16 hi + lo (two MFMAs, about 16 significant
// bits), the span / dout operand is exact; float: float MFMAs.  The bias sums
// run per thread in token order beside the staging and are combined in thread
// order; k_phi_wgrad_reduce adds the token ranges in order, so every gradient
// is the same bits on every run.
constexpr int kWgCols = 128;   // output columns per workgroup
constexpr int kWgTok = 32;     // tokens per staged chunk

template <typename T, int H>
__global__ __launch_bounds__(256) void k_phi_wgrad(const T* __restrict__ x, const T* __restrict__ dout,
                                                   const float* __restrict__ dpre, const float* __restrict__ pre,
                                                   float* __restrict__ part1, float* __restrict__ part2,
                                                   float* __restrict__ bpart1, float* __restrict__ bpart2, int BH,
                                                   int L, int D, int n, int l, int d, int ncg1, int nsplit) {
  constexpr int MT = H / 32;
  constexpr int NA = sizeof(T) == 2 ? 2 : 1;           // hi (+ lo) rows of the A operand
  constexpr int P = kWgTok + 16 / (int)sizeof(T);      // row pitch (16-byte rows, skewed banks)
  constexpr int A4 = H / 4;                            // float4 per token of dpre / pre
  constexpr int EPC = 16 / (int)sizeof(T);             // elements per 16-byte load of x / dout
  constexpr int BC = kWgCols / EPC;                    // loads per token of the column group
  static_assert(256 % A4 == 0 && kWgTok * A4 % 256 == 0 && 256 % BC == 0 && kWgTok * BC % 256 == 0,
                "fixed thread -> column slots");
  __shared__ __align__(16) T sA[NA][H][P];
  __shared__ __align__(16) T sB[kWgCols][P];
  __shared__ float sred[256][8];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, h = lane >> 5, nn = lane & 31;
  const int cg = blockIdx.x, split = blockIdx.y;
  const bool is_w2 = cg == ncg1;
  const bool want_b1 = cg == 0 && !is_w2;
  const int K = l * D;
  const int ncols = is_w2 ? D : K;
  const int col0 = is_w2 ? 0 : cg * kWgCols;
  const int64_t M = (int64_t)BH * n;
  const int64_t nchunk = (M + kWgTok - 1) / kWgTok;
  const int64_t ch0 = nchunk * split / nsplit, ch1 = nchunk * (split + 1) / nsplit;
  const float* asrc = is_w2 ? pre : dpre;
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = zero16();
  float bsum[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) bsum[j] = 0.0f;

  for (int64_t ch = ch0; ch < ch1; ++ch) {
    const int64_t g0 = ch * kWgTok;
    // A: [32 tokens][H] float -> sA[.][u][token]
#pragma unroll
    for (int j = 0; j < kWgTok * A4 / 256; ++j) {
      const int e = tid + 256 * j;
      const int tk = e / A4, u4 = e % A4;
      const int64_t g = g0 + tk;
      f32x4 v = (f32x4){0.f, 0.f, 0.f, 0.f};
      if (g < M) v = *reinterpret_cast<const f32x4*>(asrc + g * H + 4 * u4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = v[i];
        if (is_w2) a = silu_f(a);
        if (want_b1) bsum[i] += a;
        if constexpr (NA == 2) {
          const bf16 hi = (bf16)a;
          sA[0][4 * u4 + i][tk] = hi;
          sA[NA - 1][4 * u4 + i][tk] = (bf16)(a - (float)hi);
        } else {
          sA[0][4 * u4 + i][tk] = (T)a;
        }
      }
    }
    // B: [32 tokens][128 columns] of the spans (dW1) or of dout (dW2) -> sB[column][token]
#pragma unroll
    for (int j = 0; j < kWgTok * BC / 256; ++j) {
      const int e = tid + 256 * j;
      const int tk = e / BC, cc = e % BC;
      const int64_t g = g0 + tk;
      const int col = col0 + cc * EPC;
      alignas(16) T v[EPC];
#pragma unroll
      for (int q = 0; q < EPC; ++q) v[q] = (T)0.0f;
      if (g < M && col < ncols) {
        const T* src;
        if (is_w2) {
          src = dout + g * D + col;
        } else {
          const int64_t bh = g / n, i = g % n;
          src = x + (bh * L + i * d) * D + col;
        }
        *reinterpret_cast<int4*>(v) = *reinterpret_cast<const int4*>(src);
      }
#pragma unroll
      for (int q = 0; q < EPC; ++q) {
        if (is_w2) bsum[q] += to_f32(v[q]);
        sB[cc * EPC + q][tk] = v[q];
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kWgTok / 16; ++s) {
      Frag<T> b;
      b.load(&sB[32 * w + nn][16 * s + 8 * h]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int a2 = 0; a2 < NA; ++a2) {
          Frag<T> a;
          a.load(&sA[a2][32 * mt + perm32(nn)][16 * s + 8 * h]);
          mma32(acc[mt], a, b);
        }
    }
    __syncthreads();
  }

  const int col = col0 + 32 * w + nn;
  if (col < ncols) {
    float* dst = is_w2 ? part2 + (int64_t)split * H * D : part1 + (int64_t)split * H * K;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(int64_t)(32 * mt + acc_elem(h, r)) * ncols + col] = acc[mt][r];
  }
  if (want_b1 || is_w2) {   // uniform over the workgroup
#pragma unroll
    for (int j = 0; j < 8; ++j) sred[tid][j] = bsum[j];
    __syncthreads();
    if (want_b1 && tid < H) {
      // hidden unit u = 4 u4 + i: the threads with tid % A4 == u4, in thread order
      float s = 0.0f;
      for (int t = tid / 4; t < 256; t += A4) s += sred[t][tid % 4];
      bpart1[(int64_t)split * H + tid] = s;
    }
    if (is_w2 && tid < D) {
      float s = 0.0f;
      for (int t = tid / EPC; t < 256; t += BC) s += sred[t][tid % EPC];
      bpart2[(int64_t)split * D + tid] = s;
    }
  }
}

// the token ranges of k_phi_wgrad's partials added in order; one thread per
// output element of [dW1 | dpos | dW2 | db1 | db2]
__global__ __launch_bounds__(256) void k_phi_wgrad_reduce(const float* __restrict__ part1,
                                                          const float* __restrict__ part2,
                                                          const float* __restrict__ bpart1,
                                                          const float* __restrict__ bpart2,
                                                          const float* __restrict__ pos, const float* __restrict__ w1,
                                                          float* __restrict__ dw1, float* __restrict__ dpos,
                                                          float* __restrict__ dw2, float* __restrict__ db1,
                                                          float* __restrict__ db2, int H, int D, int K, int nsplit) {
  __shared__ float sdb1[128];
  for (int u = threadIdx.x; u < H; u += 256) {
    float s = 0.0f;
    for (int sp = 0; sp < nsplit; ++sp) s += bpart1[(int64_t)sp * H + u];
    sdb1[u] = s;
  }
  __syncthreads();
  int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t HK = (int64_t)H * K;
  if (e < HK) {
    const int u = (int)(e / K), k = (int)(e % K);
    float s = 0.0f;
    for (int sp = 0; sp < nsplit; ++sp) s += part1[sp * HK + e];
    dw1[e] = s + sdb1[u] * pos[k];
    return;
  }
  e -= HK;
  if (e < K) {
    float s = 0.0f;
    for (int u = 0; u < H; ++u) s += sdb1[u] * w1[(int64_t)u * K + e];
    dpos[e] = s;
    return;
  }
  e -= K;
  if (e < (int64_t)D * H) {
    const int c = (int)(e / H), u = (int)(e % H);
    float s = 0.0f;
    for (int sp = 0; sp < nsplit; ++sp) s += part2[((int64_t)sp * H + u) * D + c];
    dw2[e] = s;
    return;
  }
  e -= (int64_t)D * H;
  if (e < H) {
    db1[e] = sdb1[e];
    return;
  }
  e -= H;
  if (e < D) {
    float s = 0.0f;
    for (int sp = 0; sp < nsplit; ++sp) s += bpart2[(int64_t)sp * D + e];
    db2[e] = s;
  }
}

// token ranges of k_phi_wgrad: about two workgroups per CU of a 256-CU part,
// at least one 32-token chunk each; a function of the shape only, so the sums
// are the same bits on every device
__host__ inline int phi_wgrad_splits(int64_t M, int ncg) {
  const int64_t nchunk = (M + kWgTok - 1) / kWgTok;
  int64_t s = (512 + ncg - 1) / ncg;
  s = s < 64 ? s : 64;
  s = s < nchunk ? s : nchunk;
  return (int)(s < 1 ? 1 : s);
}

}  // namespace nsa

using namespace nsa;

extern "C" {

size_t nsa_phi_wgrad_workspace(int BH, int n, int D, int H, int l) {
  if (BH <= 0 || n <= 0 || l < 1 || (D != 64 && D != 128) || (H != 32 && H != 64 && H != 128)) return 0;
  const int K = l * D, ncg1 = (K + kWgCols - 1) / kWgCols;
  const int ns = phi_wgrad_splits((int64_t)BH * n, ncg1 + 1);
  return sizeof(float) * (size_t)ns * ((size_t)H * K + (size_t)H * D + H + D);
}

int nsa_phi_wgrad(const void* x, const void* dout, const float* dpre, const float* pre, const float* pos,
                  const float* w1, float* dw1, float* db1, float* dw2, float* db2, float* dpos, void* workspace,
                  size_t workspace_bytes, int BH, int L, int D, int H, int l, int d, int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(BH > 0 && L >= 0 && l >= 1 && d >= 1, NSA_ERR_SHAPE);
  NSA_CHECK(D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(H == 32 || H == 64 || H == 128, NSA_ERR_SHAPE);
  const int n = L >= l ? (L - l) / d + 1 : 0;
  NSA_CHECK(n > 0, NSA_ERR_SHAPE);
  NSA_CHECK(x && dout && dpre && pre && pos && w1 && dw1 && db1 && dw2 && db2 && dpos && workspace, NSA_ERR_ARG);
  const int K = l * D, ncg1 = (K + kWgCols - 1) / kWgCols;
  const int64_t M = (int64_t)BH * n;
  const int ns = phi_wgrad_splits(M, ncg1 + 1);
  NSA_CHECK(workspace_bytes >= nsa_phi_wgrad_workspace(BH, n, D, H, l), NSA_ERR_ARG);
  float* part1 = static_cast<float*>(workspace);
  float* part2 = part1 + (size_t)ns * H * K;
  float* bpart1 = part2 + (size_t)ns * H * D;
  float* bpart2 = bpart1 + (size_t)ns * H;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(ncg1 + 1, ns);
#define NSA_PHI_WGRAD(TT, HH)                                                                               \
  if (H == HH)                                                                                              \
    k_phi_wgrad<TT, HH><<<grid, 256, 0, s>>>((const TT*)x, (const TT*)dout, dpre, pre, part1, part2, bpart1, \
                                             bpart2, BH, L, D, n, l, d, ncg1, ns);
  if (dtype == NSA_BF16) {
    NSA_PHI_WGRAD(bf16, 32) NSA_PHI_WGRAD(bf16, 64) NSA_PHI_WGRAD(bf16, 128)
  } else {
    NSA_PHI_WGRAD(float, 32) NSA_PHI_WGRAD(float, 64) NSA_PHI_WGRAD(float, 128)
  }
#undef NSA_PHI_WGRAD
  const int64_t total = (int64_t)H * K + K + (int64_t)D * H + H + D;
  k_phi_wgrad_reduce<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(part1, part2, bpart1, bpart2, pos, w1, dw1,
                                                                      dpos, dw2, db1, db2, H, D, K, ns);
  return nsa_launch_status();
}

int nsa_phi_fwd(const void* x, const void* w1, const float* c1, const void* w2, const float* b2, void* out,
                float* pre, int BH, int L, int D, int H, int l, int d, int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(BH > 0 && L >= 0 && l >= 1 && d >= 1, NSA_ERR_SHAPE);
  NSA_CHECK(D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(H == 32 || H == 64 || H == 128, NSA_ERR_SHAPE);
  const int n = L >= l ? (L - l) / d + 1 : 0;
  if (n == 0) return NSA_OK;
  NSA_CHECK(x && w1 && c1 && w2 && b2 && out && pre, NSA_ERR_ARG);
  const int ntile = (n + 31) / 32;
  const int64_t grid = (int64_t)BH * ntile;   // one workgroup per 32 pooled tokens
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  hipStream_t s = (hipStream_t)stream;
#define NSA_PHI_FWD(TT, DD, HH)                                                                                    \
  if (D == DD && H == HH)                                                                                          \
    k_phi_fwd<TT, DD, HH><<<(unsigned)grid, 64 * kPhiFwdWaves, 0, s>>>((const TT*)x, (const TT*)w1, c1,           \
                                                                       (const TT*)w2, b2, (TT*)out, pre, BH, L, n, \
                                                                       l, d, ntile);
#define NSA_PHI_FWD_T(TT) \
  NSA_PHI_FWD(TT, 64, 32) NSA_PHI_FWD(TT, 64, 64) NSA_PHI_FWD(TT, 64, 128) \
  NSA_PHI_FWD(TT, 128, 32) NSA_PHI_FWD(TT, 128, 64) NSA_PHI_FWD(TT, 128, 128)
  if (dtype == NSA_BF16) {
    NSA_PHI_FWD_T(bf16)
  } else {
    NSA_PHI_FWD_T(float)
  }
#undef NSA_PHI_FWD_T
#undef NSA_PHI_FWD
  return nsa_launch_status();
}

int nsa_phi_dpre(const void* dout, const void* w2t, const float* pre, float* dpre, int BH, int n, int D, int H,
                 int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(BH > 0 && n >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(D == 64 || D == 128, NSA_ERR_SHAPE);
  NSA_CHECK(H == 32 || H == 64 || H == 128, NSA_ERR_SHAPE);
  if (n == 0) return NSA_OK;
  NSA_CHECK(dout && w2t && pre && dpre, NSA_ERR_ARG);
  const int ntile = (n + 31) / 32;
  const int64_t waves = (int64_t)BH * ntile, grid = (waves + 3) / 4;
  NSA_CHECK(grid < (1ll << 31), NSA_ERR_SHAPE);
  hipStream_t s = (hipStream_t)stream;
#define NSA_PHI_DPRE(TT, DD, HH)                                                                                   \
  if (D == DD && H == HH)                                                                                          \
    k_phi_dpre<TT, DD, HH><<<(unsigned)grid, 256, 0, s>>>((const TT*)dout, (const TT*)w2t, pre, dpre, BH, n, ntile);
#define NSA_PHI_DPRE_T(TT) \
  NSA_PHI_DPRE(TT, 64, 32) NSA_PHI_DPRE(TT, 64, 64) NSA_PHI_DPRE(TT, 64, 128) \
  NSA_PHI_DPRE(TT, 128, 32) NSA_PHI_DPRE(TT, 128, 64) NSA_PHI_DPRE(TT, 128, 128)
  if (dtype == NSA_BF16) {
    NSA_PHI_DPRE_T(bf16)
  } else {
    NSA_PHI_DPRE_T(float)
  }
#undef NSA_PHI_DPRE_T
#undef NSA_PHI_DPRE
  return nsa_launch_status();
}

int nsa_phi_fold(const void* dspan, int dspan_dtype, void* dx, int BH, int L, int D, int l, int d, int dx_dtype,
                 void* stream) {
  NSA_CHECK(dx_dtype == NSA_F32 || dx_dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(dspan_dtype == NSA_F32 || dspan_dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(BH > 0 && L >= 0 && D > 0 && l >= 1 && d >= 1, NSA_ERR_SHAPE);
  const int n = L >= l ? (L - l) / d + 1 : 0;
  NSA_CHECK(dx != nullptr && (n == 0 || dspan != nullptr), NSA_ERR_ARG);
  const int64_t total = (int64_t)BH * L * D;
  if (total == 0) return NSA_OK;
  int64_t grid = (total + 255) / 256;
  grid = grid < 65536 ? grid : 65536;
  hipStream_t s = (hipStream_t)stream;
  const bool vec8 = D % 8 == 0;   // 16-byte rows of 8 channels
  if (vec8) {
    grid = (total / 8 + 255) / 256;
    grid = grid < 65536 ? (grid < 1 ? 1 : grid) : 65536;
  }
  auto go = [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    if (vec8)
      k_phi_fold8<TI, TO><<<(unsigned)grid, 256, 0, s>>>((const TI*)dspan, (TO*)dx, BH, L, D, n, l, d);
    else
      k_phi_fold<TI, TO><<<(unsigned)grid, 256, 0, s>>>((const TI*)dspan, (TO*)dx, BH, L, D, n, l, d);
  };
  if (dspan_dtype == NSA_BF16) {
    if (dx_dtype == NSA_BF16) go(bf16{}, bf16{}); else go(bf16{}, float{});
  } else {
    if (dx_dtype == NSA_BF16) go(float{}, bf16{}); else go(float{}, float{});
  }
  return nsa_launch_status();
}

}  // extern "C"
