// Device-side building blocks shared by the NSA kernels (gfx950 / CDNA4).
//
// Every contraction runs on 16x16 MFMA tiles held by one 64-lane wave:
//   A (16 x 32, M x K): lane l holds A[l & 15][k(l >> 4, j)], j = 0..7
//   B (32 x 16, K x N): lane l holds B[k(l >> 4, j)][l & 15]
//   C (16 x 16)       : lane l holds C[4 * (l >> 4) + i][l & 15], i = 0..3
// k(g, j) is the same bijection for A and B, so any operand whose 8 slots
// per lane are filled with the same 8 K-indices on both sides contracts
// correctly.  bf16 uses one v_mfma_f32_16x16x32_bf16; fp32 issues eight
// v_mfma_f32_16x16x4_f32 (slot j of every lane forms one K=4 step), which
// keeps the per-lane operand layout identical for both element types.
//
// Attention orientation used by the query-side kernels: S^T = K Q^T with keys
// on M and the 16 query heads of one query on N, so each lane owns one head
// (column l & 15).  Key rows of a 32-key tile are permuted so that lane group
// g of the two S^T accumulators holds keys 8g .. 8g+7 of the tile; P^T then
// feeds the PV MFMA as a B operand without any data movement, and V^T / K^T
// are read as 16-byte rows of key-contiguous transposed copies.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsa {

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16;
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kMaskScore = -1.0e30f;   // finite "minus infinity" for masked scores
constexpr float kLseEmpty = -1.0e9f;      // lse sentinel of rows with no visible key
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// operand fragments: 8 elements of T per lane
// ---------------------------------------------------------------------------
template <typename T> struct Frag;

template <> struct Frag<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (bf16)0.0f;
  }
  __device__ __forceinline__ void load(const bf16* p) {
    v = *reinterpret_cast<const bf16x8*>(p);
  }
  // slots 0..3 from p0, 4..7 from p1 (two 8-byte reads)
  __device__ __forceinline__ void load2(const bf16* p0, const bf16* p1) {
    bf16x4 a = *reinterpret_cast<const bf16x4*>(p0);
    bf16x4 b = *reinterpret_cast<const bf16x4*>(p1);
    v = (bf16x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
  __device__ __forceinline__ void set(const float* x) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (bf16)x[j];
  }
  __device__ __forceinline__ bf16 elem(int j) const { return v[j]; }
  __device__ __forceinline__ void store(bf16* p) const { *reinterpret_cast<bf16x8*>(p) = v; }
};

template <> struct Frag<float> {
  f32x4 lo, hi;
  __device__ __forceinline__ void zero() {
    lo = (f32x4){0.f, 0.f, 0.f, 0.f};
    hi = lo;
  }
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4*>(p);
    hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ void load2(const float* p0, const float* p1) {
    lo = *reinterpret_cast<const f32x4*>(p0);
    hi = *reinterpret_cast<const f32x4*>(p1);
  }
  __device__ __forceinline__ void set(const float* x) {
    lo = (f32x4){x[0], x[1], x[2], x[3]};
    hi = (f32x4){x[4], x[5], x[6], x[7]};
  }
  __device__ __forceinline__ float elem(int j) const { return j < 4 ? lo[j] : hi[j - 4]; }
  __device__ __forceinline__ void store(float* p) const {
    *reinterpret_cast<f32x4*>(p) = lo;
    *reinterpret_cast<f32x4*>(p + 4) = hi;
  }
};

__device__ __forceinline__ void mma(f32x4& c, const Frag<bf16>& a, const Frag<bf16>& b) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
}

__device__ __forceinline__ void mma(f32x4& c, const Frag<float>& a, const Frag<float>& b) {
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[j], b.lo[j], c, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[j], b.hi[j], c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return (f32x4){0.f, 0.f, 0.f, 0.f}; }

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m, kWave)); }
__device__ __forceinline__ float xor_sum(float v, int m) { return v + __shfl_xor(v, m, kWave); }

// reduce across the four lane groups that share (lane & 15)
__device__ __forceinline__ float group4_max(float v) { return xor_max(xor_max(v, 16), 32); }
__device__ __forceinline__ float group4_sum(float v) { return xor_sum(xor_sum(v, 16), 32); }

// store 4 consecutive elements (one C-layout column run) as T
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
  *reinterpret_cast<bf16x4*>(p) = (bf16x4){(bf16)a, (bf16)b, (bf16)c, (bf16)d};
}
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = (f32x4){a, b, c, d};
}
__device__ __forceinline__ void store4(f16* p, float a, float b, float c, float d) {
  *reinterpret_cast<f16x4*>(p) = (f16x4){(f16)a, (f16)b, (f16)c, (f16)d};
}

// Branch outputs kept for a backward's row dots dO . o in the NSA_F16S form:
// row r holds o[r] / s_r in fp16 (11 significant bits, eight times finer than
// bf16) and the float32 scales s_r follow the rows' halves.  s_r is 1 unless
// the row's largest magnitude amax reaches 2^15 (fp16 ends at 65504); then it
// is the power of two that brings amax into [2^14, 2^15).  A power of two
// divides and multiplies back exactly, so the stored value is o[r] rounded
// once.  Infinite or NaN rows keep s_r = 1 (the values carry them).
__device__ __forceinline__ float f16s_row_scale(float amax) {
  if (!(amax >= 32768.0f) || amax == __builtin_inff()) return 1.0f;
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127;   // amax in [2^e, 2^(e+1))
  return __uint_as_float((uint32_t)(e - 14 + 127) << 23);
}
// Element type of the selection forward's partial outputs (the unnormalised
// block-local O_j = sum_k p_k v_k): fp16 for 16-bit inputs (11 significant
// bits against bf16's 8; the merged selection output, and through the row
// dot dO . o the selection dK, inherit the partials' rounding), with a
// power-of-two scale for each partial folded into its m_j (O_j / s, l_j / s,
// m_j + log2 s merge to the same output) so that rows past 2^15 stay in
// fp16's range; the input type otherwise.
template <typename T> struct PartOf { using type = T; };
template <> struct PartOf<bf16> { using type = f16; };
template <typename T> using PartT = typename PartOf<T>::type;

template <typename T> struct IsF16 { static constexpr bool value = false; };
template <> struct IsF16<f16> { static constexpr bool value = true; };

// float -> u32 with the same order (+inf highest); every float maps above 0
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Maximum (MAX) or minimum of a u32 over the wave, in every lane: within rows
// of 16 lanes by DPP (quad swaps, half-row and row mirrors), across rows by
// the gfx950 row swaps (permlane16: row pairs, permlane32: wave halves) --
// register moves only, no LDS round trips.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t x) {
  auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xF, 0xF, false));   // row_half_mirror
  x = op(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x140, 0xF, 0xF, false));   // row_mirror
  {
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = op(p[0], p[1]);   // rows 2r and 2r+1 hold their pair's result
  }
  {
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    x = op(p[0], p[1]);   // both halves: the wave's result
  }
  return x;
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Map the hardware block id to a logical one so that logically consecutive
// workgroups (neighbouring queries / the same KV head) share an XCD.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblocks) {
  constexpr int64_t kXcd = 8;
  if (nblocks < kXcd * 2) return bid;
  const int64_t per = nblocks / kXcd;           // full rows
  const int64_t full = per * kXcd;
  if (bid >= full) return bid;                  // tail keeps its id
  return (bid % kXcd) * per + bid / kXcd;
}

// Transposed K/V copies: [B*Hkv][D][Tp] with key-contiguous rows padded to Tp.
__host__ __device__ inline int padded_len(int n) { return ((n + 32 + 63) / 64) * 64; }
// The row scales of an NSA_F16S buffer: float32, after its rows * D halves.
__host__ __device__ inline float* f16s_scales(void* o, int64_t rows, int D) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(o) + rows * D * 2);
}

}  // namespace nsa
