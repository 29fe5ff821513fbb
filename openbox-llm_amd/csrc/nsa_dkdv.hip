// Key-side NSA backward: dK/dV of the range branches (window, compression) and
// of the selection branch (block-outer over the block -> query CSR).
//
// A wave owns 16 keys and walks the queries that see them two at a time
// (kv_step in nsa_tiles.h), so dK/dV stay in registers for the whole walk.
//   * window      : queries t in [k0, k0 + 15 + w - 1]; one writer per key, plain stores.
//   * compression : pooled token i is seen by every t >= i*d + l - 1; the query
//                   range is split into chunks and merged with float atomics.
//   * selection   : work items (block, chunk of its CSR query list) from
//                   nsa_sel_dkdv_items; a persistent grid drains the list and merges
//                   chunks of one block with float atomics.
#include "nsa_launch.h"
#include "nsa_tiles.h"

namespace nsa {

template <typename T>
struct KvCtx {
  const T* q;
  const T* dout;
  const T* qt;
  const T* dt;
  const float* lse;
  const float* dot;
  const float* rowscale;
  int Hq, Hkv, G, NHC, T_;
};

// Row statistics of query t for heads hc*16 + 4g + i; `vis` = key column visible to t.
template <typename T>
__device__ __forceinline__ RowStats row_stats(const KvCtx<T>& x, int b, int hkv, int hc, int t, bool tok, bool vis,
                                              int g) {
  RowStats r;
  r.vm = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hg = hc * 16 + 4 * g + i;
    const bool ok = tok && hg < x.G;
    const int64_t ri = ((int64_t)b * x.Hq + hkv * x.G + hg) * x.T_ + t;
    r.lse2[i] = ok ? x.lse[ri] * kLog2e : 0.0f;
    r.rs[i] = (ok && x.rowscale != nullptr) ? x.rowscale[ri] : 1.0f;
    r.dot[i] = ok ? x.dot[ri] : 0.0f;
    if (ok && vis) r.vm |= 1u << i;
  }
  return r;
}

// One (query A, query B) step for this wave's 16 keys; tB < 0 means no query B.
template <typename T, int D>
__device__ __forceinline__ void kv_pair(KvAcc<D>& acc, const KvCtx<T>& x, const Frag<T> (&kbf)[Dims<D>::KC],
                                        const Frag<T> (&vbf)[Dims<D>::KC], int b, int hkv, int hc, int tA, int tB,
                                        bool visA, bool visB, float sl2, int g, int c) {
  const bool hasB = tB >= 0;
  const int tb = hasB ? tB : tA;
  const int hg = hc * 16 + c;
  const bool col_ok = hg < x.G;
  const int64_t rA = ((int64_t)b * x.Hq + hkv * x.G + hg) * x.T_ + tA;
  const int64_t rB = ((int64_t)b * x.Hq + hkv * x.G + hg) * x.T_ + tb;
  const T* qA = col_ok ? x.q + rA * D : nullptr;
  const T* qB = (col_ok && hasB) ? x.q + rB * D : nullptr;
  const T* dA = col_ok ? x.dout + rA * D : nullptr;
  const T* dB = (col_ok && hasB) ? x.dout + rB * D : nullptr;
  const int64_t tbase = (((int64_t)b * x.Hkv + hkv) * x.NHC + hc) * x.T_;
  const T* qtA = x.qt + (tbase + tA) * D * 16;
  const T* qtB = x.qt + (tbase + tb) * D * 16;
  const T* dtA = x.dt + (tbase + tA) * D * 16;
  const T* dtB = x.dt + (tbase + tb) * D * 16;
  const RowStats ra = row_stats(x, b, hkv, hc, tA, true, visA, g);
  const RowStats rb = row_stats(x, b, hkv, hc, tb, hasB, visB, g);
  kv_step<T, D>(acc, kbf, vbf, qA, qB, dA, dB, qtA, qtB, dtA, dtB, ra, rb, sl2, g, c);
}

template <int D>
__device__ __forceinline__ void kv_store(const KvAcc<D>& acc, float* dk_row, float* dv_row, int g, float scale,
                                         bool atomic) {
#pragma unroll
  for (int dt = 0; dt < Dims<D>::DT; ++dt) {
    const int d0 = 16 * dt + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (atomic) {
        atomicAdd(dk_row + d0 + i, acc.dk[dt][i] * scale);
        atomicAdd(dv_row + d0 + i, acc.dv[dt][i]);
      } else {
        dk_row[d0 + i] = acc.dk[dt][i] * scale;
        dv_row[d0 + i] = acc.dv[dt][i];
      }
    }
  }
}

// Key-side B fragments: lane (g, c) holds row key (the lane's key column).
template <typename T, int D>
__device__ __forceinline__ void load_key_col(Frag<T> (&f)[Dims<D>::KC], const T* base, int key, bool ok, int g) {
  load_row_frags<T, D>(f, ok ? base + (int64_t)key * D : nullptr, g);
}

// ---------------------------------------------------------------------------
// range dK/dV
// grid: (B*Hkv) x ceil(Lk/64) x n_chunks; 4 waves, wave w owns keys k0 = 64*kt + 16*w .. +15
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void k_range_dkdv(int mode, KvCtx<T> x, const T* __restrict__ k,
                                                    const T* __restrict__ v, float* __restrict__ dk,
                                                    float* __restrict__ dv, int Lk, int nkt, int chunk, int window,
                                                    int cl, int cd, float sl2, float scale) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const int bh = blockIdx.z;
  const int kt = blockIdx.x;
  const int b = bh / x.Hkv, hkv = bh % x.Hkv;
  const int k0 = kt * 64 + w * 16;
  if (k0 >= Lk) return;
  const int key = k0 + c;
  const bool key_ok = key < Lk;
  // query range of this wave's keys
  int tlo, thi;
  if (mode == NSA_MODE_WINDOW) {
    tlo = k0;
    thi = k0 + 15 + window - 1;
  } else {
    tlo = k0 * cd + cl - 1;
    thi = x.T_ - 1;
    const int c0 = blockIdx.y * chunk;
    const int c1 = c0 + chunk - 1;
    tlo = tlo > c0 ? tlo : c0;
    thi = thi < c1 ? thi : c1;
  }
  thi = thi < x.T_ - 1 ? thi : x.T_ - 1;
  if (tlo > thi) return;
  Frag<T> kbf[Dims<D>::KC], vbf[Dims<D>::KC];
  const T* kb_ = k + (int64_t)bh * Lk * D;
  const T* vb_ = v + (int64_t)bh * Lk * D;
  load_key_col<T, D>(kbf, kb_, key, key_ok, g);
  load_key_col<T, D>(vbf, vb_, key, key_ok, g);
  KvAcc<D> acc;
  acc.init();
  for (int hc = 0; hc < x.NHC; ++hc) {
    for (int t = tlo; t <= thi; t += 2) {
      const int tB = t + 1 <= thi ? t + 1 : -1;
      bool visA, visB;
      if (mode == NSA_MODE_WINDOW) {
        visA = key_ok && key <= t && key > t - window;
        visB = tB >= 0 && key_ok && key <= tB && key > tB - window;
      } else {
        visA = key_ok && key * cd + cl - 1 <= t;
        visB = tB >= 0 && key_ok && key * cd + cl - 1 <= tB;
      }
      kv_pair<T, D>(acc, x, kbf, vbf, b, hkv, hc, t, tB, visA, visB, sl2, g, c);
    }
  }
  if (key_ok) {
    const int64_t r = ((int64_t)bh * Lk + key) * D;
    kv_store<D>(acc, dk + r, dv + r, g, scale, mode == NSA_MODE_COMPRESS);
  }
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
// selection dK/dV over CSR work items
// ---------------------------------------------------------------------------
// items[i] = {bh * n_blk + j, begin, end, 0}: pair range [begin, end) of q_of_block
__global__ __launch_bounds__(1024) void k_sel_items(const int32_t* __restrict__ offsets, int nb, int n_blk,
                                                    int chunk, int4* __restrict__ items, int32_t* __restrict__ n_items) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int per = (nb + 1023) / 1024;
  const int lo = tid * per, hi = lo + per < nb ? lo + per : nb;
  int cnt = 0;
  for (int e = lo; e < hi; ++e) {
    const int bh = e / n_blk, j = e % n_blk;
    const int n = offsets[bh * (n_blk + 1) + j + 1] - offsets[bh * (n_blk + 1) + j];
    cnt += (n + chunk - 1) / chunk;
  }
  part[tid] = cnt;
  __syncthreads();
  // Hillis-Steele inclusive scan over 1024 partial counts
  for (int off = 1; off < 1024; off <<= 1) {
    const int add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int pos = part[tid] - cnt;
  for (int e = lo; e < hi; ++e) {
    const int bh = e / n_blk, j = e % n_blk;
    const int beg = offsets[bh * (n_blk + 1) + j];
    const int end = offsets[bh * (n_blk + 1) + j + 1];
    for (int s = beg; s < end; s += chunk) {
      const int se = s + chunk < end ? s + chunk : end;
      items[pos++] = make_int4(e, s, se, 0);
    }
  }
  if (tid == 1023) *n_items = part[1023];
}

template <typename T, int D>
__global__ __launch_bounds__(256) void k_sel_dkdv(KvCtx<T> x, const T* __restrict__ k, const T* __restrict__ v,
                                                  const int32_t* __restrict__ q_of_block,
                                                  const int4* __restrict__ items, const int32_t* __restrict__ n_items,
                                                  float* __restrict__ dk, float* __restrict__ dv, int n_blk, int L,
                                                  float sl2, float scale) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c = lane & 15;
  const int ni = *n_items;
  const int nsub = L / 16;
  for (int it = blockIdx.x; it < ni; it += gridDim.x) {
    const int4 item = items[it];
    const int bh = item.x / n_blk, j = item.x % n_blk;
    const int b = bh / x.Hkv, hkv = bh % x.Hkv;
    const T* kb_ = k + (int64_t)bh * x.T_ * D;
    const T* vb_ = v + (int64_t)bh * x.T_ * D;
    for (int sub = w; sub < nsub; sub += 4) {
      const int key = j * L + sub * 16 + c;
      const bool key_ok = key < x.T_;
      Frag<T> kbf[Dims<D>::KC], vbf[Dims<D>::KC];
      load_key_col<T, D>(kbf, kb_, key, key_ok, g);
      load_key_col<T, D>(vbf, vb_, key, key_ok, g);
      KvAcc<D> acc;
      acc.init();
      for (int hc = 0; hc < x.NHC; ++hc) {
        for (int p = item.y; p < item.z; p += 2) {
          const int tA = q_of_block[p];
          const int tB = p + 1 < item.z ? q_of_block[p + 1] : -1;
          const bool visA = key_ok && key <= tA;
          const bool visB = tB >= 0 && key_ok && key <= tB;
          kv_pair<T, D>(acc, x, kbf, vbf, b, hkv, hc, tA, tB, visA, visB, sl2, g, c);
        }
      }
      if (key_ok) {
        const int64_t r = ((int64_t)bh * x.T_ + key) * D;
        kv_store<D>(acc, dk + r, dv + r, g, scale, true);
      }
    }
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

template <typename T>
static KvCtx<T> make_ctx(const void* q, const void* dout, const void* qt, const void* dt, const float* lse,
                         const float* dot, const float* rowscale, int Hq, int Hkv, int Tlen) {
  KvCtx<T> x;
  x.q = (const T*)q;
  x.dout = (const T*)dout;
  x.qt = (const T*)qt;
  x.dt = (const T*)dt;
  x.lse = lse;
  x.dot = dot;
  x.rowscale = rowscale;
  x.Hq = Hq;
  x.Hkv = Hkv;
  x.G = Hq / Hkv;
  x.NHC = (x.G + 15) / 16;
  x.T_ = Tlen;
  return x;
}

static constexpr int kCmpChunk = 1024;   // queries per compression dK/dV work item

extern "C" {

int nsa_range_dkdv(int mode, const void* q, const void* k, const void* v, const void* dout, const void* qt,
                   const void* dout_t, const float* lse, const float* dot, const float* rowscale, float* dk,
                   float* dv, int B, int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block,
                   int cmp_stride, int dtype, void* stream) {
  NSA_CHECK(mode == NSA_MODE_WINDOW || mode == NSA_MODE_COMPRESS, NSA_ERR_ARG);
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && Lk >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(mode == NSA_MODE_COMPRESS || (window >= 1 && Lk == T), NSA_ERR_SHAPE);
  NSA_CHECK(mode == NSA_MODE_WINDOW || (cmp_block >= 1 && cmp_stride >= 1), NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  hipStream_t s = (hipStream_t)stream;
  const int64_t nel = (int64_t)B * Hkv * Lk * D;
  if (mode == NSA_MODE_COMPRESS || T == 0) {
    if (zero_f32(dk, nel, s) != NSA_OK || zero_f32(dv, nel, s) != NSA_OK) return NSA_ERR_LAUNCH;
  }
  if (T == 0 || Lk == 0) return NSA_OK;
  const int nkt = (Lk + 63) / 64;
  const int nch = mode == NSA_MODE_COMPRESS ? (T + kCmpChunk - 1) / kCmpChunk : 1;
  dim3 grid(nkt, nch, B * Hkv);
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16) {
      KvCtx<bf16> x = make_ctx<bf16>(q, dout, qt, dout_t, lse, dot, rowscale, Hq, Hkv, T);
      k_range_dkdv<bf16, DD><<<grid, 256, 0, s>>>(mode, x, (const bf16*)k, (const bf16*)v, dk, dv, Lk, nkt,
                                                  kCmpChunk, window, cmp_block, cmp_stride, sl2, scale);
    } else {
      KvCtx<float> x = make_ctx<float>(q, dout, qt, dout_t, lse, dot, rowscale, Hq, Hkv, T);
      k_range_dkdv<float, DD><<<grid, 256, 0, s>>>(mode, x, (const float*)k, (const float*)v, dk, dv, Lk, nkt,
                                                   kCmpChunk, window, cmp_block, cmp_stride, sl2, scale);
    }
  });
  return nsa_launch_status();
}

// Selection blocks of the CSR consumed here: every block holding a key, the
// trailing partial one included (the forward attends to it when selected).
static inline int sel_csr_blocks(int T, int block_size) { return (T + block_size - 1) / block_size; }

static inline size_t sel_items_cap(int B, int Hkv, int T, int S, int block_size, int chunk) {
  const size_t nb = (size_t)B * Hkv * sel_csr_blocks(T, block_size);
  const size_t pairs = (size_t)B * Hkv * T * S;
  return nb + (pairs + chunk - 1) / chunk + 1;
}

size_t nsa_sel_dkdv_workspace(int B, int Hkv, int T, int S, int block_size, int chunk) {
  if (B <= 0 || Hkv <= 0 || T < 0 || S < 0 || block_size <= 0 || chunk <= 0) return 0;
  return sel_items_cap(B, Hkv, T, S, block_size, chunk) * sizeof(int4) + 256;
}

int nsa_sel_dkdv(const void* q, const void* k, const void* v, const void* dout, const void* qt, const void* dout_t,
                 const float* lse, const float* dot, const float* rowscale, const int32_t* q_of_block,
                 const int32_t* block_offsets, const int32_t* pair_count, float* dk, float* dv, void* workspace,
                 size_t workspace_bytes, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                 int dtype, void* stream) {
  (void)pair_count;
  NSA_CHECK(B > 0 && Hkv > 0 && Hq % Hkv == 0 && T >= 0 && S >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(block_size >= 16 && block_size % 16 == 0 && chunk >= 2, NSA_ERR_SHAPE);
  NSA_CHECK(dtype == NSA_F32 || dtype == NSA_BF16, NSA_ERR_DTYPE);
  NSA_CHECK(workspace_bytes >= nsa_sel_dkdv_workspace(B, Hkv, T, S, block_size, chunk), NSA_ERR_WORKSPACE);
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
  const size_t grid_cap = cap < 2048 ? cap : 2048;
  const float scale = 1.0f / sqrtf((float)D);
  const float sl2 = scale * kLog2e;
  NSA_DISPATCH_D(D, {
    if (dtype == NSA_BF16) {
      KvCtx<bf16> x = make_ctx<bf16>(q, dout, qt, dout_t, lse, dot, rowscale, Hq, Hkv, T);
      k_sel_dkdv<bf16, DD><<<(unsigned)grid_cap, 256, 0, s>>>(x, (const bf16*)k, (const bf16*)v, q_of_block, items,
                                                              n_items, dk, dv, n_blk, block_size, sl2, scale);
    } else {
      KvCtx<float> x = make_ctx<float>(q, dout, qt, dout_t, lse, dot, rowscale, Hq, Hkv, T);
      k_sel_dkdv<float, DD><<<(unsigned)grid_cap, 256, 0, s>>>(x, (const float*)k, (const float*)v, q_of_block,
                                                               items, n_items, dk, dv, n_blk, block_size, sl2,
                                                               scale);
    }
  });
  return nsa_launch_status();
}

}  // extern "C"
