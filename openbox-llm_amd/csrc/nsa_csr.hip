// Block -> query CSR on the GPU (the structure of nsa_fsa.py:14-64).
//
// Every (b, hkv, t, s) slot becomes a key (b*Hkv + hkv) * n_blk + j for a causal
// pair (j >= 0, j < n_blk, j*L <= t) and a sentinel past the last block
// otherwise; a stable LSD radix sort of (key, t) then groups the pairs by
// block with queries ascending, exactly like the reference's stable argsort.
// Offsets are lower bounds of every block key in the sorted keys.
#include <rocprim/device/device_radix_sort.hpp>

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

struct CsrLayout {
  int64_t n;
  size_t keys_in, vals_in, keys_out, temp, temp_bytes, total;
  int end_bit;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static CsrLayout csr_layout(int B, int Hkv, int T, int S, int n_blk) {
  CsrLayout c;
  c.n = (int64_t)B * Hkv * T * S;
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
