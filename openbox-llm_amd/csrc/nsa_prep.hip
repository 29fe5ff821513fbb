// Layout, pooling and gate kernels of the NSA path (all HBM-bound).
//
//  * transpose_kv   : x [BH][L][D] -> xt [BH][D][Lp]  (key-contiguous rows, zero pad)
//  * pool_fwd/bwd   : mean over spans [i*d, i*d+l)        (nsa_fused_kernel.py:549-554)
//  * gate_fwd       : out = sum_c sigmoid(g_c) o_c         (nsa_fused_kernel.py:572-573)
//  * bwd_prep       : dot_c = dO . o_c, rowscale_c = sigmoid(g_c),
//                     dgate_c = sigmoid'(g_c) dot_c        (autograd of nsa_model.py:297-301),
//                     coff_c = lse_c log2(e) - log2(rowscale_c) for the dK/dV kernels
//  * cast_f32       : fp32 accumulator -> output dtype
//  * wpool_*        : BlockCompressor's learned weighted pool and its gradients
//  * heads_split    : stacked projection -> head-major branch inputs (+ RoPE,
//                     bias), and the gradient scatter back (nsa_model.py:192-194)
#include "nsa_common.h"
#include "nsa_launch.h"

namespace nsa {

// ---------------------------------------------------------------------------
// transpose_kv: 64 x 64 tiles through LDS
// ---------------------------------------------------------------------------
// Any D and Lp: one element per access.
template <typename T>
__global__ __launch_bounds__(256) void k_transpose_kv(const T* __restrict__ x, T* __restrict__ xt,
                                                      int L, int D, int Lp) {
  __shared__ float tile[64][65];
  const int bh = blockIdx.z;
  const int l0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const T* xb = x + (int64_t)bh * L * D;
  T* yb = xt + (int64_t)bh * D * Lp;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e / 64, cc = e % 64;          // r: key, cc: d
    const int l = l0 + r, d = d0 + cc;
    tile[r][cc] = (l < L && d < D) ? to_f32(xb[(int64_t)l * D + d]) : 0.0f;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e / 64, cc = e % 64;          // r: d, cc: key
    const int d = d0 + r, l = l0 + cc;
    if (d < D && l < Lp) yb[(int64_t)d * Lp + l] = from_f32<T>(tile[cc][r]);
  }
}

// D % 8 == 0, Lp % 8 == 0, 16-byte aligned rows: 8-element global accesses.
// A lane moves 8 consecutive d of one key in, 8 consecutive keys of one d out
// (8 lanes cover a 64-element row piece).  The LDS row pitch (66 bf16 /
// 65 float) puts the 8 keys x 8 d read by a wave's lanes on distinct banks.
template <typename T>
__global__ __launch_bounds__(256) void k_transpose_kv8(const T* __restrict__ x, T* __restrict__ xt,
                                                       int L, int D, int Lp) {
  constexpr int P = sizeof(T) == 2 ? 66 : 65;
  __shared__ T tile[64 * P];
  const int bh = blockIdx.z;
  const int l0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const T* xb = x + (int64_t)bh * L * D;
  T* yb = xt + (int64_t)bh * D * Lp;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i, r = c >> 3, cc = (c & 7) * 8;   // r: key, cc: first d
    const int l = l0 + r, d = d0 + cc;
    Frag<T> f;
    if (l < L && d < D)
      f.load(xb + (int64_t)l * D + d);
    else
      f.zero();
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[r * P + cc + j] = f.elem(j);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i, r = c >> 3, kc = (c & 7) * 8;  // r: d, kc: first key
    const int d = d0 + r, l = l0 + kc;
    if (d < D && l < Lp) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = to_f32(tile[(kc + j) * P + r]);
      Frag<T> f;
      f.set(v);
      f.store(yb + (int64_t)d * Lp + l);
    }
  }
}

// ---------------------------------------------------------------------------
// pooling
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_pool_fwd(const T* __restrict__ x, T* __restrict__ out,
                                                  int BH, int L, int D, int n, int pl, int pd) {
  const int64_t total = (int64_t)BH * n * D;
  const float inv = 1.0f / (float)pl;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int d = (int)(e % D);
    const int64_t r = e / D;
    const int i = (int)(r % n);
    const int64_t bh = r / n;
    const T* src = x + (bh * L + (int64_t)i * pd) * D + d;
    float s = 0.0f;
    for (int k = 0; k < pl; ++k) s += to_f32(src[(int64_t)k * D]);
    out[e] = from_f32<T>(s * inv);
  }
}

// D % 8 == 0, 16-byte aligned rows: a lane sums 8 consecutive d (same order of
// additions as k_pool_fwd)
template <typename T>
__global__ __launch_bounds__(256) void k_pool_fwd8(const T* __restrict__ x, T* __restrict__ out,
                                                   int BH, int L, int D, int n, int pl, int pd) {
  const int dc = D / 8;
  const int64_t total = (int64_t)BH * n * dc;
  const float inv = 1.0f / (float)pl;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % dc);
    const int64_t r = e / dc;
    const int i = (int)(r % n);
    const int64_t bh = r / n;
    const T* src = x + (bh * L + (int64_t)i * pd) * D + 8 * c;
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f;
#pragma unroll 8
    for (int k = 0; k < pl; ++k) {
      Frag<T> f;
      f.load(src + (int64_t)k * D);
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] += to_f32(f.elem(j));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] *= inv;
    Frag<T> o;
    o.set(s);
    o.store(out + r * D + 8 * c);
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_pool_bwd(const TI* __restrict__ dp, TO* __restrict__ dx,
                                                  int BH, int L, int D, int n, int pl, int pd) {
  const int64_t total = (int64_t)BH * L * D;
  const float inv = 1.0f / (float)pl;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int d = (int)(e % D);
    const int64_t r = e / D;
    const int t = (int)(r % L);
    const int64_t bh = r / L;
    // tokens i with i*pd <= t < i*pd + pl
    int ilo = t - pl + 1 <= 0 ? 0 : (t - pl + 1 + pd - 1) / pd;
    int ihi = t / pd;
    if (ihi > n - 1) ihi = n - 1;
    float s = 0.0f;
    for (int i = ilo; i <= ihi; ++i) s += to_f32(dp[(bh * n + i) * D + d]);
    dx[e] = from_f32<TO>(s * inv);
  }
}

// D % 8 == 0, 16-byte aligned rows: a lane writes 8 consecutive d (same order
// of additions as k_pool_bwd)
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void k_pool_bwd8(const TI* __restrict__ dp, TO* __restrict__ dx,
                                                   int BH, int L, int D, int n, int pl, int pd) {
  const int dc = D / 8;
  const int64_t total = (int64_t)BH * L * dc;
  const float inv = 1.0f / (float)pl;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % dc);
    const int64_t r = e / dc;
    const int t = (int)(r % L);
    const int64_t bh = r / L;
    int ilo = t - pl + 1 <= 0 ? 0 : (t - pl + 1 + pd - 1) / pd;
    int ihi = t / pd;
    if (ihi > n - 1) ihi = n - 1;
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f;
    for (int i = ilo; i <= ihi; ++i) {
      Frag<TI> f;
      f.load(dp + (bh * n + i) * D + 8 * c);
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] += to_f32(f.elem(j));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] *= inv;
    Frag<TO> o;
    o.set(s);
    o.store(dx + r * D + 8 * c);
  }
}

// ---------------------------------------------------------------------------
// learned weighted pool (BlockCompressor, nsa_model.py:100-123)
// ---------------------------------------------------------------------------
// The pooled token of span i is sum_p w[p] (x[i d + p] + P[p]) for softmax
// weights w and a position code P; here sum_p w[p] x[i d + p] + cv with cv =
// w^T P, over the overlapping spans in place (no unfolded copy), in float32 as
// the module computes it.  D % 8 == 0: a lane takes 8 consecutive channels.

// out[bh][i][c] = sum_p w[p] x[bh][i d + p][c] + cv[c]   (p ascending)
template <typename T>
__global__ __launch_bounds__(256) void k_wpool_fwd8(const T* __restrict__ x, const float* __restrict__ w,
                                                    const float* __restrict__ cv, float* __restrict__ out, int BH,
                                                    int L, int D, int n, int pl, int pd) {
  const int dc = D / 8;
  const int64_t total = (int64_t)BH * n * dc;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % dc);
    const int64_t r = e / dc;
    const int i = (int)(r % n);
    const int64_t bh = r / n;
    const T* src = x + (bh * L + (int64_t)i * pd) * D + 8 * c;
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f;
#pragma unroll 8
    for (int k = 0; k < pl; ++k) {
      Frag<T> f;
      f.load(src + (int64_t)k * D);
      const float wk = w[k];
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] += wk * to_f32(f.elem(j));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] += cv[8 * c + j];
    float* o = out + r * D + 8 * c;
    *reinterpret_cast<f32x4*>(o) = (f32x4){s[0], s[1], s[2], s[3]};
    *reinterpret_cast<f32x4*>(o + 4) = (f32x4){s[4], s[5], s[6], s[7]};
  }
}

// dx[bh][t][c] = sum over the spans i that hold t (ascending) of w[t - i d] dp[bh][i][c]
template <typename TO>
__global__ __launch_bounds__(256) void k_wpool_bwd8(const float* __restrict__ dp, const float* __restrict__ w,
                                                    TO* __restrict__ dx, int BH, int L, int D, int n, int pl,
                                                    int pd) {
  const int dc = D / 8;
  const int64_t total = (int64_t)BH * L * dc;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int c = (int)(e % dc);
    const int64_t r = e / dc;
    const int t = (int)(r % L);
    const int64_t bh = r / L;
    int ilo = t - pl + 1 <= 0 ? 0 : (t - pl + 1 + pd - 1) / pd;
    int ihi = t / pd;
    if (ihi > n - 1) ihi = n - 1;
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = 0.0f;
    for (int i = ilo; i <= ihi; ++i) {
      Frag<float> g;
      g.load(dp + (bh * n + i) * D + 8 * c);
      const float wk = w[t - i * pd];
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] += wk * g.elem(j);
    }
    Frag<TO> o;
    o.set(s);
    o.store(dx + r * D + 8 * c);
  }
}

// dwp[p][bh] = sum over (i, c) of x[bh][i d + p][c] dp[bh][i][c]: workgroup
// (p, bh); thread (row lane, channel chunk) strides over the spans, then a
// tree over the workgroup (a fixed order: the same bits every run)
template <typename T>
__global__ __launch_bounds__(256) void k_wpool_dw(const T* __restrict__ x, const float* __restrict__ dp,
                                                  float* __restrict__ dwp, int BH, int L, int D, int n, int pd) {
  __shared__ float red[256];
  const int p = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int dc = D / 8, cl = tid % dc, rpi = 256 / dc;   // D / 8 divides 256 (D <= 2048)
  const T* xb = x + ((int64_t)bh * L + p) * D + 8 * cl;
  const float* gb = dp + (int64_t)bh * n * D + 8 * cl;
  float acc = 0.0f;
  for (int i = tid / dc; i < n; i += rpi) {
    Frag<T> f;
    f.load(xb + (int64_t)i * pd * D);
    Frag<float> g;
    g.load(gb + (int64_t)i * D);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += to_f32(f.elem(j)) * g.elem(j);
  }
  red[tid] = acc;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (tid < off) red[tid] += red[tid + off];
    __syncthreads();
  }
  if (tid == 0) dwp[(int64_t)p * BH + bh] = red[0];
}

// ---------------------------------------------------------------------------
// head split of a stacked projection (nsa_model.py:192-194, 325-335)
// ---------------------------------------------------------------------------
// A row of the stacked projection y [B][L][W] holds the segments one after
// another: segment k (H_k heads of hd_k channels) starts at column
// col0_k = sum_{j<k} H_j hd_j.  The split writes segment k head-major,
// out_k [B][H_k][L][hd_k], adds its bias (if any), and rotates it (if marked)
// by the half-split rotary: with h = hd / 2 and channel pairs (j, j + h),
//   o[j] = a c - b s,   o[j + h] = b c + a s,     a = x[j], b = x[j + h],
// c, s = cos, sin [t][j] from the caller's tables.  float32 arithmetic, one
// rounding to T per output.  The gradient kernel is the transpose,
//   dy[j] = g[j] c + g[j + h] s,   dy[j + h] = g[j + h] c - g[j] s,
// scattered back into the stacked row (zeros for a segment without gradient).
// Work item = (b, h, t, channel chunk), chunks fastest: head-major side
// written / read contiguously, the stacked side in 16-byte pieces per token.

constexpr int kMaxHeadSegs = 8;
struct HeadSeg {
  void* buf;            // split: out_k; gradient: d out_k or null
  const float* bias;    // split only: [H hd] float32, or null
  int col0, H, hd, rot, vec;   // vec: 8 channels per lane (else 1)
};
struct HeadSegs {
  HeadSeg s[kMaxHeadSegs];
};

// segment k (uniform over the workgroup) by constant indices into the kernel
// argument: a dynamic index would copy the table to scratch memory
__device__ __forceinline__ HeadSeg head_seg(const HeadSegs& sg, int k) {
  static_assert(kMaxHeadSegs == 8, "one case per segment");
  switch (k) {
    case 0: return sg.s[0];
    case 1: return sg.s[1];
    case 2: return sg.s[2];
    case 3: return sg.s[3];
    case 4: return sg.s[4];
    case 5: return sg.s[5];
    case 6: return sg.s[6];
    default: return sg.s[7];
  }
}

struct HeadItem {
  int64_t r, b;   // r = (b H + h) L + t
  int h, t, j0;   // j0: first channel of the item
};

__device__ __forceinline__ HeadItem head_item(int64_t e, const HeadSeg& g, int L, int nc, int step) {
  HeadItem it;
  const int c = (int)(e % nc);
  it.r = e / nc;
  it.t = (int)(it.r % L);
  const int64_t bh = it.r / L;
  it.h = (int)(bh % g.H);
  it.b = bh / g.H;
  it.j0 = c * step;
  return it;
}

__device__ __forceinline__ void load8f(const float* p, float* x) {
  const f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[j] = lo[j];
    x[4 + j] = hi[j];
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_heads_split(const T* __restrict__ y, HeadSegs sg,
                                                     const float* __restrict__ cs, const float* __restrict__ sn,
                                                     int L, int W, int B) {
  const HeadSeg g = head_seg(sg, blockIdx.y);
  T* out = (T*)g.buf;
  const int h2 = g.hd / 2, step = g.vec ? 8 : 1;
  const int nc = (g.rot ? h2 : g.hd) / step;
  const int64_t total = (int64_t)B * g.H * L * nc;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const HeadItem it = head_item(e, g, L, nc, step);
    const T* src = y + (it.b * L + it.t) * W + g.col0 + it.h * g.hd;
    T* dst = out + it.r * g.hd;
    const float* bias = g.bias ? g.bias + it.h * g.hd : nullptr;
    if (g.vec) {
      float a[8], b[8], c[8], s[8];
      Frag<T> fa;
      fa.load(src + it.j0);
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = to_f32(fa.elem(j)) + (bias ? bias[it.j0 + j] : 0.0f);
      if (g.rot) {
        Frag<T> fb;
        fb.load(src + h2 + it.j0);
        load8f(cs + (int64_t)it.t * h2 + it.j0, c);
        load8f(sn + (int64_t)it.t * h2 + it.j0, s);
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          b[j] = to_f32(fb.elem(j)) + (bias ? bias[h2 + it.j0 + j] : 0.0f);
          o[j] = a[j] * c[j] - b[j] * s[j];
          b[j] = b[j] * c[j] + a[j] * s[j];
        }
        fa.set(o);
        fa.store(dst + it.j0);
        fb.set(b);
        fb.store(dst + h2 + it.j0);
      } else {
        fa.set(a);
        fa.store(dst + it.j0);
      }
    } else {
      const int j = it.j0;
      const float a = to_f32(src[j]) + (bias ? bias[j] : 0.0f);
      if (g.rot) {
        const float b = to_f32(src[h2 + j]) + (bias ? bias[h2 + j] : 0.0f);
        const float c = cs[(int64_t)it.t * h2 + j], s = sn[(int64_t)it.t * h2 + j];
        dst[j] = from_f32<T>(a * c - b * s);
        dst[h2 + j] = from_f32<T>(b * c + a * s);
      } else {
        dst[j] = from_f32<T>(a);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_heads_merge_grad(T* __restrict__ dy, HeadSegs sg,
                                                          const float* __restrict__ cs,
                                                          const float* __restrict__ sn, int L, int W, int B,
                                                          int nseg, int wseg) {
  if ((int)blockIdx.y == nseg) {   // padding columns [wseg, W): zero gradient
    const int pw = W - wseg;
    const int64_t total = (int64_t)B * L * pw;
    for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256)
      dy[(e / pw) * W + wseg + (int)(e % pw)] = from_f32<T>(0.0f);
    return;
  }
  const HeadSeg g = head_seg(sg, blockIdx.y);
  const T* gin = (const T*)g.buf;
  const int h2 = g.hd / 2, step = g.vec ? 8 : 1;
  const int nc = (g.rot ? h2 : g.hd) / step;
  const int64_t total = (int64_t)B * g.H * L * nc;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const HeadItem it = head_item(e, g, L, nc, step);
    T* dst = dy + (it.b * L + it.t) * W + g.col0 + it.h * g.hd;
    const T* src = gin ? gin + it.r * g.hd : nullptr;
    if (g.vec) {
      float a[8], b[8], c[8], s[8];
      Frag<T> fa, fb;
      if (src) {
        fa.load(src + it.j0);
        if (g.rot) fb.load(src + h2 + it.j0);
      } else {
        fa.zero();
        fb.zero();
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) a[j] = to_f32(fa.elem(j));
      if (g.rot) {
        load8f(cs + (int64_t)it.t * h2 + it.j0, c);
        load8f(sn + (int64_t)it.t * h2 + it.j0, s);
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          b[j] = to_f32(fb.elem(j));
          o[j] = a[j] * c[j] + b[j] * s[j];
          b[j] = b[j] * c[j] - a[j] * s[j];
        }
        fa.set(o);
        fa.store(dst + it.j0);
        fb.set(b);
        fb.store(dst + h2 + it.j0);
      } else {
        fa.set(a);
        fa.store(dst + it.j0);
      }
    } else {
      const int j = it.j0;
      const float a = src ? to_f32(src[j]) : 0.0f;
      if (g.rot) {
        const float b = src ? to_f32(src[h2 + j]) : 0.0f;
        const float c = cs[(int64_t)it.t * h2 + j], s = sn[(int64_t)it.t * h2 + j];
        dst[j] = from_f32<T>(a * c + b * s);
        dst[h2 + j] = from_f32<T>(b * c - a * s);
      } else {
        dst[j] = from_f32<T>(a);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// gate
// ---------------------------------------------------------------------------

// 16-byte vectors of T: 8 bf16 or 4 float
template <typename T> struct Vec16;
template <> struct Vec16<bf16> {
  static constexpr int N = 8;
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ float operator[](int i) const { return (float)v[i]; }
  __device__ __forceinline__ void set(int i, float x) { v[i] = (bf16)x; }
  __device__ __forceinline__ void store(bf16* p) const { *reinterpret_cast<bf16x8*>(p) = v; }
  __device__ __forceinline__ void store_nt(bf16* p) const {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(__builtin_bit_cast(u4, v), reinterpret_cast<u4*>(p));
  }
};
template <> struct Vec16<float> {
  static constexpr int N = 4;
  f32x4 v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const f32x4*>(p); }
  __device__ __forceinline__ float operator[](int i) const { return v[i]; }
  __device__ __forceinline__ void set(int i, float x) { v[i] = x; }
  __device__ __forceinline__ void store(float* p) const { *reinterpret_cast<f32x4*>(p) = v; }
  __device__ __forceinline__ void store_nt(float* p) const { __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p)); }
};

// One thread per 16-byte vector of the output (D is a multiple of the vector).
template <typename T>
__global__ __launch_bounds__(256) void k_gate_fwd(const T* __restrict__ g, const T* __restrict__ oc,
                                                  const T* __restrict__ os, const T* __restrict__ ow,
                                                  T* __restrict__ out, int64_t rows, int D) {
  constexpr int N = Vec16<T>::N;
  const int vpr = D / N;
  const int64_t total = rows * vpr;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / vpr;
    const float g0 = sigmoidf(to_f32(g[r * 3 + 0]));
    const float g1 = sigmoidf(to_f32(g[r * 3 + 1]));
    const float g2 = sigmoidf(to_f32(g[r * 3 + 2]));
    Vec16<T> a, b, c, y;
    a.load(oc + e * N);
    b.load(os + e * N);
    c.load(ow + e * N);
#pragma unroll
    for (int i = 0; i < N; ++i) y.set(i, g0 * a[i] + g1 * b[i] + g2 * c[i]);
    y.store(out + e * N);
  }
}

// A group of D / N lanes per row (N = elements per 16-byte vector), each
// lane one vector; 64 / (D / N) rows per wave.  nbr = number of branches
// (1: plain delta, 3: gated three-branch prep).
// N consecutive branch-output elements as float: TO is the input type (one
// Vec16) or float kept unrounded by the forward (N / 4 16-byte loads).
template <typename T, typename TO> struct BranchRow {
  static constexpr int N = Vec16<T>::N;
  float x[N];
  __device__ __forceinline__ void load(const TO* p) {
    if constexpr (IsF16<TO>::value) {
      static_assert(N == 8, "NSA_F16S rows pair with 16-bit inputs");
      const f16x8 v = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
      for (int i = 0; i < N; ++i) x[i] = (float)v[i];
    } else if constexpr (sizeof(TO) == sizeof(T)) {
      Vec16<T> v;
      v.load(reinterpret_cast<const T*>(p));
#pragma unroll
      for (int i = 0; i < N; ++i) x[i] = v[i];
    } else {
#pragma unroll
      for (int c = 0; c < N / 4; ++c) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p + 4 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * c + i] = v[i];
      }
    }
  }
};

template <typename T, typename TO>
__global__ __launch_bounds__(256) void k_bwd_prep(const T* __restrict__ dout, const TO* __restrict__ o0,
                                                  const TO* __restrict__ o1, const TO* __restrict__ o2,
                                                  const T* __restrict__ gate, T* __restrict__ dgate,
                                                  const float* __restrict__ lse0, const float* __restrict__ lse1,
                                                  const float* __restrict__ lse2, float* __restrict__ dot,
                                                  float* __restrict__ rowscale, float* __restrict__ coff,
                                                  T* __restrict__ dout_packed, int G, int T_, int64_t rows, int D,
                                                  int nbr, float* __restrict__ dgate32) {
  constexpr int N = Vec16<T>::N;
  const int gs = D / N;                         // lanes per row, a power of two <= 64
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / gs;
  const int sub = lane & (gs - 1);
  const bool ok = row < rows;
  float acc[3] = {0.f, 0.f, 0.f};
  // row (b, hkv G + g, t) -> packed row ((b Hkv + hkv) T + t) G + g
  int64_t prow = row;
  if (dout_packed != nullptr) {
    const int64_t bhq = row / T_;
    prow = ((bhq / G) * T_ + (row - bhq * T_)) * G + bhq % G;
  }
  // the tail operands of the branches this lane finishes (c = sub, sub + gs,
  // ...: one each once gs >= 3), fetched before the rows so that their
  // latency overlaps the rows'
  float gv[3], lv[3], sv[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int c = sub + k * gs;
    gv[k] = 0.0f;
    lv[k] = 0.0f;
    sv[k] = 1.0f;
    if (ok && c < nbr) {
      if (nbr == 3) gv[k] = to_f32(gate[row * 3 + c]);
      if (coff) lv[k] = (c == 0 ? lse0 : c == 1 ? lse1 : lse2)[row];
      // NSA_F16S: the rows were stored divided by their power-of-two scales
      if constexpr (IsF16<TO>::value)
        sv[k] = f16s_scales(const_cast<TO*>(c == 0 ? o0 : c == 1 ? o1 : o2), rows, D)[row];
    }
  }
  if (ok) {
    Vec16<T> d;
    BranchRow<T, TO> x;
    d.load(dout + row * D + sub * N);
    // the packed copy, read by a later launch: rows of 128 bytes or more
    // fill whole lines and skip the cache (shorter ones share lines with rows
    // that other instructions write, so they keep the cached store)
    if (dout_packed != nullptr) {
      if (D * (int)sizeof(T) >= 128)
        d.store_nt(dout_packed + prow * D + sub * N);
      else
        d.store(dout_packed + prow * D + sub * N);
    }
    const TO* os[3] = {o0, o1, o2};
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if (c >= nbr) break;
      x.load(os[c] + row * D + sub * N);
#pragma unroll
      for (int i = 0; i < N; ++i) acc[c] += d[i] * x.x[i];
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c)
    for (int m = 1; m < gs; m <<= 1) acc[c] += __shfl_xor(acc[c], m, kWave);
  if (!ok || sub >= nbr) return;
  // with dout_packed, the statistics of the selection branch (the only
  // branch, or branch 1 of 3) go to the packed row, the layout of the
  // selection dK/dV's query side
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int c = sub + k * gs;
    if (c >= nbr) break;
    const float a = (c == 0 ? acc[0] : c == 1 ? acc[1] : acc[2]) * sv[k];
    if (nbr == 1) {
      dot[prow] = a;
      if (coff) coff[prow] = lv[k] * kLog2e;
      continue;
    }
    const float sg = sigmoidf(gv[k]);
    const int64_t sr = c == 1 ? prow : row;
    dot[(int64_t)c * rows + sr] = a;
    rowscale[(int64_t)c * rows + sr] = sg;
    if (coff) coff[(int64_t)c * rows + sr] = lv[k] * kLog2e - __log2f(sg);
    if (dgate32) dgate32[row * 3 + c] = sg * (1.0f - sg) * a;
    else if (dgate) dgate[row * 3 + c] = from_f32<T>(sg * (1.0f - sg) * a);
  }
}

// [B, Hkv*G, T, D] -> [B, Hkv, T, G, D] in 16-byte chunks, 2^cs per row:
// workgroup r = (b, hkv, t) writes the G contiguous rows of query t.
__global__ __launch_bounds__(256) void k_pack_heads(const uint4* __restrict__ src, uint4* __restrict__ dst, int G,
                                                    int T, int cs, int64_t rows) {
  const int n = G << cs;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t bh = r / T;
    const int t = (int)(r - bh * T);
    const uint4* sp = src + ((bh * G * T + t) << cs);   // head 0 of the group
    uint4* dp = dst + r * n;
    for (int i = threadIdx.x; i < n; i += 256) {
      const int g = i >> cs, c = i & ((1 << cs) - 1);
      dp[i] = sp[(((int64_t)g * T) << cs) + c];
    }
  }
}

// x, y 16-byte aligned: 8 elements per access for the first n & ~7, the rest one by one
template <typename T>
__global__ __launch_bounds__(256) void k_cast_f32(const float* __restrict__ x, T* __restrict__ y, int64_t n) {
  const int64_t n8 = n >> 3;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n8; e += (int64_t)gridDim.x * 256) {
    Frag<float> f;
    f.load(x + 8 * e);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = f.elem(j);
    Frag<T> o;
    o.set(v);
    o.store(y + 8 * e);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const int64_t e = (n8 << 3) + threadIdx.x;
    y[e] = from_f32<T>(x[e]);
  }
}

// any alignment
template <typename T>
__global__ __launch_bounds__(256) void k_cast_f32_1(const float* __restrict__ x, T* __restrict__ y, int64_t n) {
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) y[e] = from_f32<T>(x[e]);
}

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static inline int grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

// The segment table of a split / gradient call, checked: segments fill the
// row from column 0 (*wseg columns; the rest of the W-column pitch is
// padding), rotated ones share one even head dim (the tables' width).  The
// vector path needs 16-byte aligned pieces.  Returns NSA_OK or an error;
// *items = the largest segment's work items (the grid's x extent).
static int head_segs(HeadSegs& sg, void* const* bufs, const float* const* biases, const int* heads,
                     const int* head_dim, const int* rotate, int nseg, const float* cos_t, const float* sin_t,
                     int B, int T, int W, const void* stacked, bool need_bufs, int64_t* items, int* wseg) {
  NSA_CHECK(nseg >= 1 && nseg <= kMaxHeadSegs && heads && head_dim && rotate && bufs, NSA_ERR_ARG);
  NSA_CHECK(B > 0 && T >= 0 && W > 0, NSA_ERR_SHAPE);
  NSA_CHECK(T == 0 || stacked, NSA_ERR_ARG);   // empty tensors may hold null pointers
  int64_t col = 0;
  int rot_hd = 0;
  *items = 0;
  for (int k = 0; k < nseg; ++k) {
    const int H = heads[k], hd = head_dim[k], rot = rotate[k] ? 1 : 0;
    NSA_CHECK(H > 0 && hd > 0, NSA_ERR_SHAPE);
    NSA_CHECK(!need_bufs || T == 0 || bufs[k], NSA_ERR_ARG);
    if (rot) {
      NSA_CHECK(hd % 2 == 0 && (rot_hd == 0 || rot_hd == hd), NSA_ERR_SHAPE);
      NSA_CHECK(cos_t && sin_t, NSA_ERR_ARG);
      rot_hd = hd;
    }
    HeadSeg& g = sg.s[k];
    g.buf = bufs[k];
    g.bias = biases ? biases[k] : nullptr;
    g.col0 = (int)col;
    g.H = H;
    g.hd = hd;
    g.rot = rot;
    g.vec = hd % (rot ? 16 : 8) == 0 && col % 8 == 0 && W % 8 == 0 && aligned16(stacked) &&
            (!bufs[k] || aligned16(bufs[k])) && (!rot || (aligned16(cos_t) && aligned16(sin_t)));
    const int64_t per = (rot ? hd / 2 : hd) / (g.vec ? 8 : 1);
    const int64_t n = (int64_t)B * H * T * per;
    if (n > *items) *items = n;
    col += (int64_t)H * hd;
    NSA_CHECK(col <= W, NSA_ERR_SHAPE);
  }
  *wseg = (int)col;   // columns [col, W) are padding
  for (int k = nseg; k < kMaxHeadSegs; ++k) sg.s[k] = sg.s[0];
  return NSA_OK;
}

}  // namespace nsa

using namespace nsa;

extern "C" {

int nsa_transpose_kv(const void* x, void* xt, int BH, int L, int D, int Lp, int dtype, void* stream) {
  NSA_CHECK(BH > 0 && L >= 0 && D > 0 && Lp >= L, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  if (L == 0 && Lp == 0) return NSA_OK;
  dim3 grid((Lp + 63) / 64, (D + 63) / 64, BH);
  hipStream_t s = (hipStream_t)stream;
  const bool vec = D % 8 == 0 && Lp % 8 == 0 && aligned16(x) && aligned16(xt);
  if (dtype == NSA_BF16) {
    if (vec)
      k_transpose_kv8<bf16><<<grid, 256, 0, s>>>((const bf16*)x, (bf16*)xt, L, D, Lp);
    else
      k_transpose_kv<bf16><<<grid, 256, 0, s>>>((const bf16*)x, (bf16*)xt, L, D, Lp);
  } else {
    if (vec)
      k_transpose_kv8<float><<<grid, 256, 0, s>>>((const float*)x, (float*)xt, L, D, Lp);
    else
      k_transpose_kv<float><<<grid, 256, 0, s>>>((const float*)x, (float*)xt, L, D, Lp);
  }
  return nsa_launch_status();
}

int nsa_pool_fwd(const void* x, void* out, int B, int H, int T, int D, int l, int d, int dtype,
                 void* stream) {
  NSA_CHECK(B > 0 && H > 0 && T >= 0 && D > 0 && l > 0 && d > 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  const int n = T >= l ? (T - l) / d + 1 : 0;
  const int64_t total = (int64_t)B * H * n * D;
  if (total == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (D % 8 == 0 && aligned16(x) && aligned16(out)) {
    const int g = grid_for(total / 8);
    if (dtype == NSA_BF16)
      k_pool_fwd8<bf16><<<g, 256, 0, s>>>((const bf16*)x, (bf16*)out, B * H, T, D, n, l, d);
    else
      k_pool_fwd8<float><<<g, 256, 0, s>>>((const float*)x, (float*)out, B * H, T, D, n, l, d);
  } else if (dtype == NSA_BF16) {
    k_pool_fwd<bf16><<<grid_for(total), 256, 0, s>>>((const bf16*)x, (bf16*)out, B * H, T, D, n, l, d);
  } else {
    k_pool_fwd<float><<<grid_for(total), 256, 0, s>>>((const float*)x, (float*)out, B * H, T, D, n, l, d);
  }
  return nsa_launch_status();
}

// dpool_dtype: dtype of the pooled-gradient input (fp32 accumulators or the model dtype)
int nsa_pool_bwd(const void* dpool, int dpool_dtype, void* dx, int B, int H, int T, int D, int l, int d,
                 int dtype, void* stream) {
  NSA_CHECK(B > 0 && H > 0 && T >= 0 && D > 0 && l > 0 && d > 0, NSA_ERR_SHAPE);
  NSA_CHECK((dtype == NSA_F32 || dtype == NSA_BF16) && (dpool_dtype == NSA_F32 || dpool_dtype == NSA_BF16),
            NSA_ERR_DTYPE);
  const int n = T >= l ? (T - l) / d + 1 : 0;
  const int64_t total = (int64_t)B * H * T * D;
  if (total == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (D % 8 == 0 && aligned16(dpool) && aligned16(dx)) {
    const int g = grid_for(total / 8);
    if (dpool_dtype == NSA_F32) {
      if (dtype == NSA_BF16)
        k_pool_bwd8<float, bf16><<<g, 256, 0, s>>>((const float*)dpool, (bf16*)dx, B * H, T, D, n, l, d);
      else
        k_pool_bwd8<float, float><<<g, 256, 0, s>>>((const float*)dpool, (float*)dx, B * H, T, D, n, l, d);
    } else {
      if (dtype == NSA_BF16)
        k_pool_bwd8<bf16, bf16><<<g, 256, 0, s>>>((const bf16*)dpool, (bf16*)dx, B * H, T, D, n, l, d);
      else
        k_pool_bwd8<bf16, float><<<g, 256, 0, s>>>((const bf16*)dpool, (float*)dx, B * H, T, D, n, l, d);
    }
    return nsa_launch_status();
  }
  const int grid = grid_for(total);
  if (dpool_dtype == NSA_F32) {
    if (dtype == NSA_BF16)
      k_pool_bwd<float, bf16><<<grid, 256, 0, s>>>((const float*)dpool, (bf16*)dx, B * H, T, D, n, l, d);
    else
      k_pool_bwd<float, float><<<grid, 256, 0, s>>>((const float*)dpool, (float*)dx, B * H, T, D, n, l, d);
  } else {
    if (dtype == NSA_BF16)
      k_pool_bwd<bf16, bf16><<<grid, 256, 0, s>>>((const bf16*)dpool, (bf16*)dx, B * H, T, D, n, l, d);
    else
      k_pool_bwd<bf16, float><<<grid, 256, 0, s>>>((const bf16*)dpool, (float*)dx, B * H, T, D, n, l, d);
  }
  return nsa_launch_status();
}

int nsa_wpool_fwd(const void* x, const float* w, const float* cvec, float* out, int B, int H, int T, int D, int l,
                  int d, int dtype, void* stream) {
  NSA_CHECK(B > 0 && H > 0 && T >= 0 && D > 0 && D % 8 == 0 && l > 0 && d > 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  const int n = T >= l ? (T - l) / d + 1 : 0;
  const int64_t total = (int64_t)B * H * n * D;
  if (total == 0) return NSA_OK;
  NSA_CHECK(x && w && cvec && out && aligned16(x) && aligned16(out), NSA_ERR_ARG);
  hipStream_t s = (hipStream_t)stream;
  const int g = grid_for(total / 8);
  if (dtype == NSA_BF16)
    k_wpool_fwd8<bf16><<<g, 256, 0, s>>>((const bf16*)x, w, cvec, out, B * H, T, D, n, l, d);
  else
    k_wpool_fwd8<float><<<g, 256, 0, s>>>((const float*)x, w, cvec, out, B * H, T, D, n, l, d);
  return nsa_launch_status();
}

int nsa_wpool_bwd(const float* dpool, const float* w, void* dx, int B, int H, int T, int D, int l, int d, int dtype,
                  void* stream) {
  NSA_CHECK(B > 0 && H > 0 && T >= 0 && D > 0 && D % 8 == 0 && l > 0 && d > 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  const int n = T >= l ? (T - l) / d + 1 : 0;
  const int64_t total = (int64_t)B * H * T * D;
  if (total == 0) return NSA_OK;
  NSA_CHECK(w && dx && aligned16(dx) && (n == 0 || (dpool && aligned16(dpool))), NSA_ERR_ARG);
  hipStream_t s = (hipStream_t)stream;
  const int g = grid_for(total / 8);
  if (dtype == NSA_BF16)
    k_wpool_bwd8<bf16><<<g, 256, 0, s>>>(dpool, w, (bf16*)dx, B * H, T, D, n, l, d);
  else
    k_wpool_bwd8<float><<<g, 256, 0, s>>>(dpool, w, (float*)dx, B * H, T, D, n, l, d);
  return nsa_launch_status();
}

int nsa_wpool_dw(const void* x, const float* dpool, float* dw_part, int B, int H, int T, int D, int l, int d,
                 int dtype, void* stream) {
  NSA_CHECK(B > 0 && H > 0 && T >= 0 && D > 0 && D % 8 == 0 && D <= 2048 && l > 0 && d > 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK((int64_t)B * H < 65536, NSA_ERR_SHAPE);   // the grid's second dimension
  const int n = T >= l ? (T - l) / d + 1 : 0;
  NSA_CHECK(x && dw_part && aligned16(x) && (n == 0 || (dpool && aligned16(dpool))), NSA_ERR_ARG);
  hipStream_t s = (hipStream_t)stream;
  // n == 0: every part is an empty sum, written as 0 by the kernel's loop
  const dim3 grid((unsigned)l, (unsigned)(B * H));
  if (dtype == NSA_BF16)
    k_wpool_dw<bf16><<<grid, 256, 0, s>>>((const bf16*)x, dpool, dw_part, B * H, T, D, n, d);
  else
    k_wpool_dw<float><<<grid, 256, 0, s>>>((const float*)x, dpool, dw_part, B * H, T, D, n, d);
  return nsa_launch_status();
}

int nsa_heads_split(const void* y, void* const* outs, const float* const* biases, const int* heads,
                    const int* head_dim, const int* rotate, int nseg, const float* cos_t, const float* sin_t, int B,
                    int T, int W, int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  HeadSegs sg;
  int64_t items = 0;
  int wseg = 0;
  const int rc =
      head_segs(sg, outs, biases, heads, head_dim, rotate, nseg, cos_t, sin_t, B, T, W, y, true, &items, &wseg);
  if (rc != NSA_OK) return rc;
  if (items == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)grid_for(items), (unsigned)nseg);
  if (dtype == NSA_BF16)
    k_heads_split<bf16><<<grid, 256, 0, s>>>((const bf16*)y, sg, cos_t, sin_t, T, W, B);
  else
    k_heads_split<float><<<grid, 256, 0, s>>>((const float*)y, sg, cos_t, sin_t, T, W, B);
  return nsa_launch_status();
}

int nsa_heads_merge_grad(const void* const* douts, void* dy, const int* heads, const int* head_dim,
                         const int* rotate, int nseg, const float* cos_t, const float* sin_t, int B, int T, int W,
                         int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  HeadSegs sg;
  int64_t items = 0;
  int wseg = 0;
  const int rc = head_segs(sg, const_cast<void* const*>(douts), nullptr, heads, head_dim, rotate, nseg, cos_t, sin_t,
                           B, T, W, dy, false, &items, &wseg);
  if (rc != NSA_OK) return rc;
  if (items == 0) return NSA_OK;
  const int64_t pad_items = (int64_t)B * T * (W - wseg);
  if (pad_items > items) items = pad_items;
  hipStream_t s = (hipStream_t)stream;
  // one more workgroup row zeroes the padding columns
  const dim3 grid((unsigned)grid_for(items), (unsigned)(nseg + (W > wseg ? 1 : 0)));
  if (dtype == NSA_BF16)
    k_heads_merge_grad<bf16><<<grid, 256, 0, s>>>((bf16*)dy, sg, cos_t, sin_t, T, W, B, nseg, wseg);
  else
    k_heads_merge_grad<float><<<grid, 256, 0, s>>>((float*)dy, sg, cos_t, sin_t, T, W, B, nseg, wseg);
  return nsa_launch_status();
}

int nsa_gate_fwd(const void* gate, const void* o_cmp, const void* o_slc, const void* o_win, void* out,
                 int64_t rows, int D, int dtype, void* stream) {
  NSA_CHECK(rows >= 0 && D > 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(D % 8 == 0, NSA_ERR_SHAPE);
  const int64_t total = rows * (D / (dtype == NSA_BF16 ? 8 : 4));
  if (total == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NSA_BF16)
    k_gate_fwd<bf16><<<grid_for(total), 256, 0, s>>>((const bf16*)gate, (const bf16*)o_cmp, (const bf16*)o_slc,
                                                     (const bf16*)o_win, (bf16*)out, rows, D);
  else
    k_gate_fwd<float><<<grid_for(total), 256, 0, s>>>((const float*)gate, (const float*)o_cmp,
                                                      (const float*)o_slc, (const float*)o_win, (float*)out,
                                                      rows, D);
  return nsa_launch_status();
}

// rows = B*Hq*T.  nbr == 1 and gate == NULL: dot[r] = dO.o0 (plain delta).
// nbr == 3: dot[c*rows + r], rowscale[c*rows + r] = sigmoid(gate[r,c]), dgate[r,c].
// coff (nullable): lse_c * log2(e) - log2(rowscale_c), laid out like dot.
// dout_packed (nullable): dO in the [B][Hkv][T][G][D] layout; the statistics
// of the selection branch (nbr == 1: the only branch, nbr == 3: branch 1) are
// then written at the packed row ((b Hkv + hkv) T + t) G + g instead of r.
int nsa_bwd_prep(const void* dout, const void* o0, const void* o1, const void* o2, const void* gate,
                 void* dgate, const float* lse0, const float* lse1, const float* lse2, float* dot,
                 float* rowscale, float* coff, void* dout_packed, int G, int T, int64_t rows, int D, int nbr,
                 int dtype, int o_dtype, int dgate_dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(o_dtype == dtype || o_dtype == NSA_F32 || (o_dtype == NSA_F16S && dtype == NSA_BF16), NSA_ERR_DTYPE);
  NSA_CHECK(dgate_dtype == dtype || dgate_dtype == NSA_F32, NSA_ERR_DTYPE);
  float* dgate32 = dgate_dtype == NSA_F32 && dtype != NSA_F32 ? (float*)dgate : nullptr;
  if (dgate32 != nullptr) dgate = nullptr;
  const int vec = dtype == NSA_BF16 ? 8 : 4;
  NSA_CHECK(rows >= 0 && D > 0 && D % vec == 0 && (nbr == 1 || nbr == 3), NSA_ERR_SHAPE);
  const int gs = D / vec;
  NSA_CHECK(gs <= 64 && (gs & (gs - 1)) == 0, NSA_ERR_SHAPE);
  NSA_CHECK(nbr == 1 || (gate && o1 && o2 && rowscale), NSA_ERR_ARG);
  NSA_CHECK(!coff || (lse0 && (nbr == 1 || (lse1 && lse2))), NSA_ERR_ARG);
  NSA_CHECK(!dout_packed || (G >= 1 && T >= 1 && rows % ((int64_t)G * T) == 0 && dout_packed != dout),
            NSA_ERR_ARG);
  if (rows == 0) return NSA_OK;
  const int64_t grid64 = (rows * gs + 255) / 256;
  NSA_CHECK(grid64 < (1ll << 31), NSA_ERR_SHAPE);
  const int grid = (int)grid64;
  hipStream_t s = (hipStream_t)stream;
  if (o_dtype == NSA_F16S)
    k_bwd_prep<bf16, f16><<<grid, 256, 0, s>>>((const bf16*)dout, (const f16*)o0, (const f16*)o1,
                                               (const f16*)o2, (const bf16*)gate, (bf16*)dgate, lse0, lse1, lse2,
                                               dot, rowscale, coff, (bf16*)dout_packed, G, T, rows, D, nbr, dgate32);
  else if (dtype == NSA_BF16 && o_dtype == NSA_BF16)
    k_bwd_prep<bf16, bf16><<<grid, 256, 0, s>>>((const bf16*)dout, (const bf16*)o0, (const bf16*)o1,
                                                (const bf16*)o2, (const bf16*)gate, (bf16*)dgate, lse0, lse1, lse2,
                                                dot, rowscale, coff, (bf16*)dout_packed, G, T, rows, D, nbr, dgate32);
  else if (dtype == NSA_BF16)
    k_bwd_prep<bf16, float><<<grid, 256, 0, s>>>((const bf16*)dout, (const float*)o0, (const float*)o1,
                                                 (const float*)o2, (const bf16*)gate, (bf16*)dgate, lse0, lse1,
                                                 lse2, dot, rowscale, coff, (bf16*)dout_packed, G, T, rows, D, nbr,
                                                 dgate32);
  else
    k_bwd_prep<float, float><<<grid, 256, 0, s>>>((const float*)dout, (const float*)o0, (const float*)o1,
                                                  (const float*)o2, (const float*)gate, (float*)dgate, lse0, lse1,
                                                  lse2, dot, rowscale, coff, (float*)dout_packed, G, T, rows, D,
                                                  nbr, nullptr);
  return nsa_launch_status();
}

int nsa_pack_heads(const void* src, void* dst, int B, int Hkv, int G, int T, int D, int dtype, void* stream) {
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(B >= 0 && Hkv >= 0 && G > 0 && T >= 0, NSA_ERR_SHAPE);
  const int bytes = D * (dtype == NSA_BF16 ? 2 : 4);
  NSA_CHECK(D > 0 && bytes % 16 == 0, NSA_ERR_SHAPE);
  NSA_CHECK(src != dst, NSA_ERR_ARG);
  const int ch = bytes / 16;
  NSA_CHECK((ch & (ch - 1)) == 0 && (int64_t)G * ch < (1ll << 31), NSA_ERR_SHAPE);
  const int64_t rows = (int64_t)B * Hkv * T;
  if (rows == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int grid = rows < 65536 ? (int)rows : 65536;
  k_pack_heads<<<grid, 256, 0, s>>>((const uint4*)src, (uint4*)dst, G, T, __builtin_ctz(ch), rows);
  return nsa_launch_status();
}

int nsa_cast_f32(const float* x, void* y, int64_t n, int dtype, void* stream) {
  NSA_CHECK(n >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  if (n == 0) return NSA_OK;
  hipStream_t s = (hipStream_t)stream;
  if (aligned16(x) && aligned16(y)) {
    const int g = grid_for(n / 8);
    if (dtype == NSA_BF16)
      k_cast_f32<bf16><<<g, 256, 0, s>>>(x, (bf16*)y, n);
    else
      k_cast_f32<float><<<g, 256, 0, s>>>(x, (float*)y, n);
  } else if (dtype == NSA_BF16) {
    k_cast_f32_1<bf16><<<grid_for(n), 256, 0, s>>>(x, (bf16*)y, n);
  } else {
    k_cast_f32_1<float><<<grid_for(n), 256, 0, s>>>(x, (float*)y, n);
  }
  return nsa_launch_status();
}

}  // extern "C"
