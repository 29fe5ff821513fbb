// Work items of the block-outer selection kernels: (block, chunk of its CSR
// query list), built on the GPU from the CSR offsets.  Shared by the
// selection forward (nsa_selbo.hip) and dK/dV (nsa_dkdv.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsa {

// items[i] = {bh * n_blk + j, begin, end, 0}: pair range [begin, end) of q_of_block;
// n_items[0] = item count, n_items[1] = 0 (the work counter of next_item).
// The items of block e are items[first[e] .. first[e + 1]), in query order
// (first: nb + 1 ints, optional).
static __global__ __launch_bounds__(1024) void k_sel_items(const int32_t* __restrict__ offsets, int nb, int n_blk,
                                                           int chunk, int4* __restrict__ items,
                                                           int32_t* __restrict__ n_items,
                                                           int32_t* __restrict__ first = nullptr) {
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
    if (first != nullptr) first[e] = pos;
    for (int s = beg; s < end; s += chunk) {
      const int se = s + chunk < end ? s + chunk : end;
      items[pos++] = make_int4(e, s, se, 0);
    }
  }
  if (tid == 1023) {
    n_items[0] = part[1023];
    n_items[1] = 0;
    if (first != nullptr) first[nb] = part[1023];
  }
}

// Next work item of a persistent grid over `total` items: the first
// gridDim.x go to the workgroups in order, each later one to the workgroup
// that asks first (the hardware dispatches workgroups as slots free up, so
// both halves balance dynamically).  Called by every thread of the workgroup
// after a barrier that follows its last read of *slot.
__device__ __forceinline__ int next_item(int32_t* counter, int* slot) {
  if (threadIdx.x == 0) *slot = (int)gridDim.x + atomicAdd(counter, 1);
  __syncthreads();
  return *slot;
}

// Selection blocks of the CSR consumed by the block-outer kernels: every
// block holding a key, the trailing partial one included (the forward attends
// to it when selected).
__host__ __device__ inline int sel_csr_blocks(int T, int block_size) { return (T + block_size - 1) / block_size; }

static inline size_t sel_items_cap(int B, int Hkv, int T, int S, int block_size, int chunk) {
  const size_t nb = (size_t)B * Hkv * sel_csr_blocks(T, block_size);
  const size_t pairs = (size_t)B * Hkv * T * S;
  return nb + (pairs + chunk - 1) / chunk + 1;
}

// Most CSR entries in one selection work item (the kernels stage an item's
// entries in LDS); the item chunk passed to the entry points is capped here.
constexpr int kSelItemMax = 1024;

// Keys of a selection block handled per pass of the block-outer kernels; a
// block longer than this is split into ceil(L / kSelPass) partial slots.
constexpr int kSelPass = 64;

// Largest GQA group whose selection row tiles hold floor(32 / G) >= 3 entries
// (G heads each) instead of two queries x 16 head slots.
constexpr int kGroupPackMaxG = 10;
__host__ __device__ inline int sel_passes(int block_size) { return (block_size + kSelPass - 1) / kSelPass; }

// Packed (query, slot) entries of the CSR built with pack_slot:
// (t << sel_slot_bits(S)) | s, so that the kernels split them with a shift
// and a mask; they sort like (t, s).
__host__ __device__ inline int sel_slot_bits(int S) {
  int b = 0;
  while ((1 << b) < S) ++b;
  return b;
}

// Slot of a selected block j in row t is valid (has a CSR pair) iff
// 0 <= j < n_csr and j * L <= t.
__device__ __forceinline__ bool sel_slot_valid(int j, int n_csr, int L, int t) {
  return j >= 0 && j < n_csr && (int64_t)j * L <= t;
}

}  // namespace nsa
