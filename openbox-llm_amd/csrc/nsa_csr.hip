// Block -> query CSR on the GPU (the structure of nsa_fsa.py:14-64).
//
// Every (b, hkv, t, s) slot with a causal pair (j >= 0, j < n_blk, j*L <= t)
// goes to the list of key (b*Hkv + hkv) * n_blk + j; lists in key order, each
// with its pairs in input order ((t, s) ascending), exactly like the
// reference's stable argsort.  Two builds give the same arrays:
//
//  * counting (LDS for 3 n_blk + 64 S ints): one wave per chunk of 64 queries of
//    one (b, hkv) counts its pairs per block in LDS; an exclusive scan over the
//    counts in (key, chunk) order gives every chunk's first slot in every
//    list; the wave then places its pairs, a pair's rank in its list within
//    the chunk being the number of earlier queries of the chunk on its block
//    (a 64-bit query mask per block).  Deterministic, no atomics outside LDS,
//    no memsets.
//  * sort (otherwise): a stable LSD radix sort of (key, value) with a
//    sentinel key for the non-causal slots; offsets are lower bounds of the
//    keys in the sorted keys.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include "nsa_launch.h"
#include "nsa_items.h"

namespace nsa {

// vals: the query t, or (t << sel_slot_bits(S)) | s (s: the slot of the pair in
// block_idx) when pack_slot
__global__ __launch_bounds__(256) void k_csr_keys(const int32_t* __restrict__ idx, uint32_t* __restrict__ keys,
                                                  int32_t* __restrict__ vals, int64_t n, int T, int S, int n_blk,
                                                  int L, uint32_t sentinel, int pack_slot) {
  const int sbits = sel_slot_bits(S);
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / S;
    const int t = (int)(r % T);
    const int64_t bh = r / T;
    const int j = idx[e];
    const bool ok = j >= 0 && j < n_blk && (int64_t)j * L <= t;
    keys[e] = ok ? (uint32_t)(bh * n_blk + j) : sentinel;
    vals[e] = pack_slot ? (t << sbits) | (int)(e % S) : t;
  }
}

__device__ __forceinline__ int64_t lower_bound_u32(const uint32_t* a, int64_t n, uint32_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (a[mid] < x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(256) void k_csr_offsets(const uint32_t* __restrict__ skeys, int64_t n, int nbh,
                                                     int n_blk, int32_t* __restrict__ offsets,
                                                     int32_t* __restrict__ count) {
  const int64_t total = (int64_t)nbh * (n_blk + 1);
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int bh = (int)(e / (n_blk + 1));
    const int j = (int)(e % (n_blk + 1));
    offsets[e] = (int32_t)lower_bound_u32(skeys, n, (uint32_t)(bh * n_blk + j));
  }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    *count = (int32_t)lower_bound_u32(skeys, n, (uint32_t)((int64_t)nbh * n_blk));
}

__global__ __launch_bounds__(256) void k_csr_pair_bh(const uint32_t* __restrict__ skeys, const int32_t* __restrict__ count,
                                                     int32_t* __restrict__ pair_bh, int64_t n, int n_blk) {
  const int64_t P = *count;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256)
    pair_bh[e] = e < P ? (int32_t)(skeys[e] / (uint32_t)n_blk) : -1;
}

// The stable radix sort of the (key, value) pairs.  rocprim sorts up to
// MergeSortLimit items by block sort + merge passes (about 10 passes at 2^20
// pairs); past the limit by onesweep LSD passes over the few key bits.  The
// limit is lowered so that the CSR's sizes (2^17 pairs and up) take onesweep.
// Both algorithms are stable: equal keys keep the input order.
using CsrSortConfig = rocprim::radix_sort_config<rocprim::default_config, rocprim::default_config,
                                                 rocprim::default_config, (size_t)1 << 17>;

static inline hipError_t csr_sort(void* temp, size_t& bytes, const uint32_t* kin, uint32_t* kout, const int32_t* vin,
                                  int32_t* vout, int n, int end_bit, hipStream_t s) {
  return rocprim::radix_sort_pairs<CsrSortConfig>(temp, bytes, kin, kout, vin, vout, n, 0u, (unsigned)end_bit, s);
}

// ---- counting build ---------------------------------------------------------
constexpr int kCsrChunkQ = 64;            // queries per chunk (one wave)
constexpr int kCsrCountLds = 64 * 1024;   // LDS bytes per wave

// The chunk's block indices with all loads in flight at once (16 a lane per
// batch), then handed to f(i, raw index) in input order per lane.
template <typename F>
__device__ __forceinline__ void csr_chunk_loads(const int32_t* __restrict__ idx, int64_t e0, int ne, int lane, F f) {
  for (int b0 = 0; b0 < ne; b0 += 16 * 64) {
    int v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = b0 + k * 64 + lane;
      v[k] = i < ne ? idx[e0 + i] : -1;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = b0 + k * 64 + lane;
      if (i < ne) f(i, v[k]);
    }
  }
}

// LDS per-list counters of one chunk: 16 loads a lane in flight per batch
__device__ __forceinline__ void csr_lds_rows(int* __restrict__ dst, const int32_t* __restrict__ src, int n_blk,
                                             int nchunk, int lane) {
  for (int b0 = 0; b0 < n_blk; b0 += 16 * 64) {
    int v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int j = b0 + k * 64 + lane;
      v[k] = j < n_blk ? src[(int64_t)j * nchunk] : 0;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int j = b0 + k * 64 + lane;
      if (j < n_blk) dst[j] = v[k];
    }
  }
}

__device__ __forceinline__ bool csr_causal(int j, int t, int n_blk, int L) {
  return j >= 0 && j < n_blk && (int64_t)j * L <= t;
}

// counts[(bh n_blk + j) nchunk + c] = pairs of chunk c of bh on block j
__global__ __launch_bounds__(64) void k_csr_count(const int32_t* __restrict__ idx, int32_t* __restrict__ counts,
                                                  int T, int S, int n_blk, int L, int nchunk) {
  extern __shared__ int cnt[];
  const int c = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  for (int j = lane; j < n_blk; j += 64) cnt[j] = 0;
  __syncthreads();
  const int t0 = c * kCsrChunkQ;
  const int ne = min(kCsrChunkQ, T - t0) * S;
  const int64_t e0 = ((int64_t)bh * T + t0) * S;
  csr_chunk_loads(idx, e0, ne, lane, [&](int i, int j) {
    if (csr_causal(j, t0 + i / S, n_blk, L)) atomicAdd(&cnt[j], 1);
  });
  __syncthreads();
  int32_t* out = counts + (int64_t)bh * n_blk * nchunk + c;
  for (int j = lane; j < n_blk; j += 64) out[(int64_t)j * nchunk] = cnt[j];
}

// LDS of the place kernel, in ints: list slots run[n_blk], query masks
// mask[n_blk] (64-bit), the chunk's indices stage[64 S], a duplicate flag
__host__ __device__ inline int64_t csr_place_lds_ints(int n_blk, int S) {
  const int64_t r = ((int64_t)n_blk + 1) & ~(int64_t)1;   // masks 8-byte aligned
  return r + 2 * (int64_t)n_blk + (int64_t)kCsrChunkQ * S + 2;
}

// pos = exclusive scan of counts: the chunk's first slot in each list.  Lane
// q takes query t0 + q: its S indices are staged in LDS and its bit set in the
// 64-bit query mask of each of its blocks.  A pair of query q on block j then
// lands at run[j] + popcount(mask[j] & bits below q): the pairs of block j
// from earlier queries of the chunk come first.  A row holding one block
// twice (an atomicOr that finds its bit already set) makes the chunk take the
// exact walk instead: pairs in input order, 64 a slice, each slot its list's
// running slot plus the earlier lanes of the slice on the same block (ballot
// per distinct block of the slice).
__global__ __launch_bounds__(64) void k_csr_place(const int32_t* __restrict__ idx, const int32_t* __restrict__ pos,
                                                  int32_t* __restrict__ q_of_block, int32_t* __restrict__ pair_bh,
                                                  int T, int S, int n_blk, int L, int nchunk, int pack_slot) {
  extern __shared__ int run[];
  uint64_t* mask = (uint64_t*)(run + (((int64_t)n_blk + 1) & ~(int64_t)1));
  int* stage = (int*)(mask + n_blk);
  int* dup = stage + kCsrChunkQ * S;
  const int c = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  const int t0 = c * kCsrChunkQ;
  const int nq = min(kCsrChunkQ, T - t0);
  const int ne = nq * S;
  const int64_t e0 = ((int64_t)bh * T + t0) * S;
  const int sbits = sel_slot_bits(S);
  for (int j = lane; j < n_blk; j += 64) mask[j] = 0;
  if (lane == 0) *dup = 0;
  csr_lds_rows(run, pos + (int64_t)bh * n_blk * nchunk + c, n_blk, nchunk, lane);
  csr_chunk_loads(idx, e0, ne, lane, [&](int i, int j) { stage[i] = j; });
  __syncthreads();
  const int t = t0 + lane;
  if (lane < nq) {
    bool twice = false;
    for (int sl = 0; sl < S; ++sl) {
      const int j = stage[lane * S + sl];
      if (csr_causal(j, t, n_blk, L)) {
        const uint64_t old = atomicOr((unsigned long long*)&mask[j], 1ull << lane);
        twice |= ((old >> lane) & 1ull) != 0;
      }
    }
    if (twice) *dup = 1;
  }
  __syncthreads();
  if (*dup == 0) {
    if (lane < nq) {
      const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
      for (int sl = 0; sl < S; ++sl) {
        const int j = stage[lane * S + sl];
        if (csr_causal(j, t, n_blk, L)) {
          const int p = run[j] + __popcll(mask[j] & below);
          q_of_block[p] = pack_slot ? (t << sbits) | sl : t;
          if (pair_bh) pair_bh[p] = bh;
        }
      }
    }
    return;
  }
  for (int i0 = 0; i0 < ne; i0 += 64) {
    const int i = i0 + lane;
    const int ti = t0 + i / S, sl = i % S;
    int j = -1;
    if (i < ne) {
      const int b = stage[i];
      if (csr_causal(b, ti, n_blk, L)) j = b;
    }
    int before = 0, cnt = 0;
    for (uint64_t todo = __ballot(j >= 0); todo != 0;) {   // uniform loop over the slice's blocks
      const int lk = __builtin_amdgcn_readlane(j, __builtin_ctzll(todo));
      const uint64_t m = __ballot(j == lk);
      if (j == lk) {
        before = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        cnt = __popcll(m);
      }
      todo &= ~m;
    }
    if (j >= 0) {
      const int base = run[j];
      const int p = base + before;
      q_of_block[p] = pack_slot ? (ti << sbits) | sl : ti;
      if (pair_bh) pair_bh[p] = bh;
      if (before == cnt - 1) run[j] = base + cnt;   // the slice's last pair on block j
    }
    __syncthreads();
  }
}

// offsets[bh][j] = first slot of list (bh, j) (j = n_blk: the end of bh's
// lists), *count = number of pairs, tails of q_of_block / pair_bh = -1
__global__ __launch_bounds__(256) void k_csr_finish(const int32_t* __restrict__ counts,
                                                    const int32_t* __restrict__ pos, int64_t M, int nbh, int n_blk,
                                                    int nchunk, int32_t* __restrict__ offsets,
                                                    int32_t* __restrict__ count, int32_t* __restrict__ q_of_block,
                                                    int32_t* __restrict__ pair_bh, int64_t cap) {
  const int32_t total = M > 0 ? pos[M - 1] + counts[M - 1] : 0;
  const int64_t noff = (int64_t)nbh * (n_blk + 1);
  const int64_t n = noff > cap ? noff : cap;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    if (e < noff) {
      const int bh = (int)(e / (n_blk + 1)), j = (int)(e % (n_blk + 1));
      const int64_t k = (int64_t)bh * n_blk + j;   // j == n_blk: the next bh's first list
      offsets[e] = (M > 0 && k < (int64_t)nbh * n_blk) ? pos[k * nchunk] : total;
    }
    if (e >= total && e < cap) {
      q_of_block[e] = -1;
      if (pair_bh) pair_bh[e] = -1;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) *count = total;
}

static inline hipError_t csr_scan(void* temp, size_t& bytes, const int32_t* in, int32_t* out, int64_t M,
                                  hipStream_t s) {
  return rocprim::exclusive_scan(temp, bytes, in, out, (int32_t)0, (size_t)M, rocprim::plus<int32_t>(), s);
}

// ---- layout of the workspace -----------------------------------------------------
struct CsrLayout {
  int64_t n;
  bool counting;
  int nchunk;
  int64_t M;               // counting: nbh * n_blk * nchunk
  size_t keys_in, vals_in, keys_out, temp, temp_bytes, total;
  int end_bit;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static CsrLayout csr_layout(int B, int Hkv, int T, int S, int n_blk) {
  CsrLayout c;
  c.n = (int64_t)B * Hkv * T * S;
  c.nchunk = (T + kCsrChunkQ - 1) / kCsrChunkQ;
  c.M = (int64_t)B * Hkv * n_blk * c.nchunk;
  c.counting = csr_place_lds_ints(n_blk, S) * 4 <= kCsrCountLds && c.M < (1ll << 31) &&
               (int64_t)B * Hkv <= 65535;   // grid y: B*Hkv
  c.end_bit = 0;
  if (c.counting) {
    // keys_in: counts [M], vals_in: pos [M], temp: the scan's storage
    c.temp_bytes = 0;
    (void)csr_scan(nullptr, c.temp_bytes, nullptr, nullptr, c.M, (hipStream_t)0);
    c.keys_in = 0;
    c.vals_in = c.keys_in + align256(c.M * sizeof(int32_t));
    c.keys_out = c.vals_in + align256(c.M * sizeof(int32_t));
    c.temp = c.keys_out;
    c.total = c.temp + align256(c.temp_bytes) + 256;
    return c;
  }
  const uint64_t sentinel = (uint64_t)B * Hkv * n_blk;
  int bits = 1;
  while (bits < 32 && (1ull << bits) <= sentinel) ++bits;
  c.end_bit = bits;
  c.temp_bytes = 0;
  (void)csr_sort(nullptr, c.temp_bytes, nullptr, nullptr, nullptr, nullptr, (int)c.n, c.end_bit, (hipStream_t)0);
  c.keys_in = 0;
  c.vals_in = c.keys_in + align256(c.n * sizeof(uint32_t));
  c.keys_out = c.vals_in + align256(c.n * sizeof(int32_t));
  c.temp = c.keys_out + align256(c.n * sizeof(uint32_t));
  c.total = c.temp + align256(c.temp_bytes) + 256;
  return c;
}

static inline int grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace nsa

using namespace nsa;

extern "C" {

size_t nsa_csr_workspace(int B, int Hkv, int T, int S, int n_blk) {
  if (B <= 0 || Hkv <= 0 || T < 0 || S < 0 || n_blk < 0) return 0;
  if ((int64_t)B * Hkv * T * S >= (1ll << 31) || (int64_t)B * Hkv * n_blk >= (1ll << 31)) return 0;
  return csr_layout(B, Hkv, T, S, n_blk).total;
}

int nsa_csr_build(const int32_t* block_idx, int32_t* q_of_block, int32_t* block_offsets, int32_t* pair_bh,
                  int32_t* pair_count, void* workspace, size_t workspace_bytes, int B, int Hkv, int T, int S,
                  int block_size, int n_blk, int pack_slot, void* stream) {
  NSA_CHECK(B > 0 && Hkv > 0 && T >= 0 && S >= 0 && block_size > 0 && n_blk >= 0, NSA_ERR_SHAPE);
  NSA_CHECK(!pack_slot || ((int64_t)T << sel_slot_bits(S)) < (1ll << 31), NSA_ERR_SHAPE);
  NSA_CHECK((int64_t)B * Hkv * T * S < (1ll << 31) && (int64_t)B * Hkv * n_blk < (1ll << 31), NSA_ERR_SHAPE);
  const CsrLayout c = csr_layout(B, Hkv, T, S, n_blk);
  NSA_CHECK(workspace_bytes >= c.total, NSA_ERR_WORKSPACE);
  hipStream_t s = (hipStream_t)stream;
  const int nbh = B * Hkv;
  char* ws = (char*)workspace;
  uint32_t* kin = (uint32_t*)(ws + c.keys_in);
  int32_t* vin = (int32_t*)(ws + c.vals_in);
  uint32_t* kout = (uint32_t*)(ws + c.keys_out);
  void* temp = ws + c.temp;
  if (c.counting) {
    const size_t lds_count = (size_t)(n_blk > 0 ? n_blk : 1) * sizeof(int);
    const size_t lds = (size_t)csr_place_lds_ints(n_blk, S) * sizeof(int);
    int32_t* counts = (int32_t*)(ws + c.keys_in);
    int32_t* pos = (int32_t*)(ws + c.vals_in);
    if (c.M > 0) {
      const dim3 grid((unsigned)c.nchunk, (unsigned)nbh);
      k_csr_count<<<grid, 64, lds_count, s>>>(block_idx, counts, T, S, n_blk, block_size, c.nchunk);
      if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
      size_t tb = c.temp_bytes;
      if (csr_scan(temp, tb, counts, pos, c.M, s) != hipSuccess) return NSA_ERR_LAUNCH;
      k_csr_place<<<grid, 64, lds, s>>>(block_idx, pos, q_of_block, pair_bh, T, S, n_blk, block_size, c.nchunk,
                                        pack_slot);
      if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
    }
    const int64_t nfin = std::max<int64_t>((int64_t)nbh * (n_blk + 1), c.n);
    k_csr_finish<<<grid_for(nfin), 256, 0, s>>>(counts, pos, c.M, nbh, n_blk, c.nchunk, block_offsets, pair_count,
                                                 q_of_block, pair_bh, c.n);
    if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
    return NSA_OK;
  }
  if (c.n > 0) {
    k_csr_keys<<<grid_for(c.n), 256, 0, s>>>(block_idx, kin, vin, c.n, T, S, n_blk, block_size,
                                             (uint32_t)((int64_t)nbh * n_blk), pack_slot);
    if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
    size_t tb = c.temp_bytes;
    if (csr_sort(temp, tb, kin, kout, vin, q_of_block, (int)c.n, c.end_bit, s) != hipSuccess) return NSA_ERR_LAUNCH;
  }
  k_csr_offsets<<<grid_for((int64_t)nbh * (n_blk + 1)), 256, 0, s>>>(kout, c.n, nbh, n_blk, block_offsets,
                                                                     pair_count);
  if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
  if (c.n > 0 && pair_bh != nullptr && n_blk > 0) {
    k_csr_pair_bh<<<grid_for(c.n), 256, 0, s>>>(kout, pair_count, pair_bh, c.n, n_blk);
    if (hipGetLastError() != hipSuccess) return NSA_ERR_LAUNCH;
  }
  return NSA_OK;
}

}  // extern "C"
