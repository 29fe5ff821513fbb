// 32x32 MFMA tiles and LDS staging shared by the LDS-tiled NSA kernels
// (range forward / dQ, and the key-side dK/dV kernel).
//
// One 32x32 MFMA per 16-deep contraction step (bf16: v_mfma_f32_32x32x16_bf16;
// fp32: eight v_mfma_f32_32x32x2f32 over the same 8 slots per lane):
//   A (32 x 16): lane (h = lane >> 5, m = lane & 31) holds A[m][slot(h, j)], j = 0..7
//   B (16 x 32): lane (h, n) holds B[slot(h, j)][n]
//   C (32 x 32): lane (h, n) register r holds C[8 (r >> 2) + 4 h + (r & 3)][n]
// slot(h, j) is the same bijection on both operands, so a fragment only has
// to hold the same 8 contraction indices on the A and B side.
//
// Operand rows are permuted inside a 32-row tile by perm32 (bits 2 and 3 of
// the row swapped).  Accumulator registers 8s .. 8s+7 of lane half h then hold
// tile elements 16s + 8h .. 16s + 8h + 7, which is exactly the B-operand
// fragment of contraction step s over that tile: an S^T (or S) accumulator is
// converted to the next MFMA's operand without moving data between lanes.
//
// LDS tiles are unpadded and filled by direct global -> LDS loads
// (global_load_lds_dwordx4: lane i of a wave writes LDS base + 16 i).  Their
// 16-byte chunks are XOR-swizzled per row so that the fragment reads of a
// wave hit distinct banks:
//   row tile    [32][D]: logical chunk c of row r sits at c ^ rkey(r).  With
//                        16 or more chunks per row rkey(r) = 4 (r & 3) +
//                        ((r >> 2) & 3): the 16 rows 16 adjacent lanes read
//                        (perm32 or natural order) get 16 distinct keys, and
//                        the 4 consecutive rows of a transposed read
//                        (lds_tr_frag, 4 chunks each) keys 4 apart, so its
//                        16 pieces per 256 bytes are distinct.  Shorter rows:
//                        rkey(r) = 2 (r & 3) + bit 3 of r, masked
//   column tile [D][32]: logical chunk c of row d sits at c ^ ckey(d)
//
// Transposed operands (a contraction over the tile's rows) come straight from
// a row tile through ds_read_b64_tr_b16: within each group of 16 lanes, lane
// l receives element (l & 3) of the 8-byte pieces addressed by lanes
// 4j + (l >> 2), j = 0..3 (measured on gfx950).
#pragma once

#include <type_traits>

#include "nsa_common.h"

namespace nsa {

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ void mma32(f32x16& c, const Frag<bf16>& a, const Frag<bf16>& b) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, c, 0, 0, 0);
}

__device__ __forceinline__ void mma32(f32x16& c, const Frag<float>& a, const Frag<float>& b) {
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[j], b.lo[j], c, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[j], b.hi[j], c, 0, 0, 0);
}

// operand row m of a 32-row tile reads tile element perm32(m)
__device__ __forceinline__ int perm32(int m) { return (m & 0x13) | ((m & 4) << 1) | ((m & 8) >> 1); }

// tile element held by accumulator register r of lane half h (after perm32)
__device__ __forceinline__ int acc_elem(int h, int r) { return 16 * (r >> 3) + 8 * h + (r & 7); }

template <typename T, int D> struct Tile32 {
  static constexpr int KS = D / 16;                        // 16-deep contraction steps over D
  static constexpr int DT = (D + 31) / 32;                 // 32-row tiles over D
  static constexpr int EPC = 16 / (int)sizeof(T);          // elements per 16-byte chunk
  static constexpr int RCH = D * (int)sizeof(T) / 16;      // chunks per row of a row tile
  static constexpr int CCH = 32 * (int)sizeof(T) / 16;     // chunks per row of a column tile
  static constexpr int ROW_ELEMS = 32 * D;                 // one [32][D] tile
  static constexpr int COL_ELEMS = D * 32;                 // one [D][32] tile
  static constexpr int ROW_CHUNKS = 32 * RCH;
  static constexpr int COL_CHUNKS = D * CCH;
  // gfx950 serves a 16-byte-per-lane LDS read 16 lanes (256 bytes, every
  // bank once) at a time: the keys give the rows that 16 adjacent lanes read
  // distinct chunks (rows sharing a 256-byte line: the same key, different
  // halves or quarters of the line)
  static __device__ __forceinline__ int rkey(int r) {
    return RCH >= 16 ? 4 * (r & 3) + ((r >> 2) & 3) : (((r & 3) << 1) | ((r >> 3) & 1)) & (RCH - 1);
  }
  // row tiles read in natural row order (lanes 0..15 read rows 0..15)
  static __device__ __forceinline__ int nkey(int r) { return (RCH >= 16 ? r : r / (16 / RCH)) & (RCH - 1); }
  static __device__ __forceinline__ int ckey(int d) { return (d / (16 / CCH)) & (CCH - 1); }
};

// A fragment of a [32][D] row tile: permuted row, contraction step s
template <typename T, int D>
__device__ __forceinline__ void lds_row_frag(Frag<T>& f, const T* tile, int m, int h, int s) {
  using C = Tile32<T, D>;
  const int r = perm32(m);
  const T* row = tile + r * D;
  const int c0 = (16 * s + 8 * h) / C::EPC;
  if (sizeof(T) == 2)
    f.load(row + (c0 ^ C::rkey(r)) * C::EPC);
  else
    f.load2(row + (c0 ^ C::rkey(r)) * C::EPC, row + ((c0 + 1) ^ C::rkey(r)) * C::EPC);
}

// B fragment of a [32][D] row tile read in natural row order (swizzled by
// nkey): lane (h, n) holds row n, elements 16s + 8h .. 16s + 8h + 7
template <typename T, int D>
__device__ __forceinline__ void lds_nrow_frag(Frag<T>& f, const T* tile, int n, int h, int s) {
  using C = Tile32<T, D>;
  const T* row = tile + n * D;
  const int c0 = (16 * s + 8 * h) / C::EPC;
  if (sizeof(T) == 2)
    f.load(row + (c0 ^ C::nkey(n)) * C::EPC);
  else
    f.load2(row + (c0 ^ C::nkey(n)) * C::EPC, row + ((c0 + 1) ^ C::nkey(n)) * C::EPC);
}

// A fragment of a [D][32] column tile: row 32dt + m (zero past D), step s
template <typename T, int D>
__device__ __forceinline__ void lds_col_frag(Frag<T>& f, const T* tile, int dt, int m, int h, int s) {
  using C = Tile32<T, D>;
  const int d = 32 * dt + m;
  if (D % 32 == 0 || d < D) {
    const T* row = tile + d * 32;
    const int c0 = (16 * s + 8 * h) / C::EPC;
    if (sizeof(T) == 2)
      f.load(row + (c0 ^ C::ckey(d)) * C::EPC);
    else
      f.load2(row + (c0 ^ C::ckey(d)) * C::EPC, row + ((c0 + 1) ^ C::ckey(d)) * C::EPC);
  } else {
    f.zero();
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16.  Kernels that fill LDS with the builtin DMA
// (__builtin_amdgcn_global_load_lds) get a full vmcnt wait in front of this
// read from the compiler; the asm DMA of lds_dma16 / lds_dma4 does not.
__device__ __forceinline__ s16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// A use of the fragment's registers: the compiler completes the loads that
// produce them here rather than at a later first use.
template <typename T>
__device__ __forceinline__ void settle(Frag<T>& f) {
  if constexpr (sizeof(T) == 2)
    asm volatile("" : "+v"(f.v));
  else
    asm volatile("" : "+v"(f.lo), "+v"(f.hi));
}

// Transposed operand from a [32][D] row tile (natural row order, rkey
// swizzle): lane (h, m) holds tile[16 s + 8 h + j][32 dt + m], j = 0..7 --
// the A operand of a product contracting over the tile's rows, slot-matched
// to the accumulator-as-B fragments of the same rows.  Columns past D (D < 32)
// repeat earlier columns and only feed accumulator rows that are never stored.
template <typename T, int D>
__device__ __forceinline__ void lds_tr_frag(Frag<T>& f, const T* tile, int dt, int lane, int s) {
  using C = Tile32<T, D>;
  if constexpr (sizeof(T) == 2) {
    // two 4-row transposed reads; source lane (g, jj, q) addresses row
    // 16 s + 8 (g >> 1) + 4 rd + jj, columns 32 dt + 16 (g & 1) + 4 q .. + 3
    const int g = lane >> 4, jj = (lane >> 2) & 3, q = lane & 3;
    int col = 32 * dt + 16 * (g & 1) + 4 * q;
    if (D % 32 != 0) col = col < D - 4 ? col : D - 4;
    const int ch = col / C::EPC, off = col % C::EPC;
    s16x4 r[2];
#pragma unroll
    for (int rd = 0; rd < 2; ++rd) {
      const int row = 16 * s + 8 * (g >> 1) + 4 * rd + jj;
      r[rd] = lds_read_tr16(tile + row * D + (ch ^ C::rkey(row)) * C::EPC + off);
    }
    const s16x4 a = r[0], b = r[1];
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 v = (s16x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    f.v = __builtin_bit_cast(bf16x8, v);
  } else {
    // float: eight single-element reads (lanes of a row read consecutive columns)
    const int h = lane >> 5;
    int col = 32 * dt + (lane & 31);
    if (D % 32 != 0) col = col < D ? col : D - 1;
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = 16 * s + 8 * h + j;
      x[j] = tile[row * D + ((col / C::EPC) ^ C::rkey(row)) * C::EPC + col % C::EPC];
    }
    f.set(x);
  }
}

// Physical chunk P of a row tile -> (row, logical chunk)
template <typename T, int D>
__device__ __forceinline__ void row_chunk(int P, int& r, int& c) {
  using C = Tile32<T, D>;
  r = P / C::RCH;
  c = (P % C::RCH) ^ C::rkey(r);
}

// Physical chunk P of a natural-order row tile -> (row, logical chunk)
template <typename T, int D>
__device__ __forceinline__ void nrow_chunk(int P, int& r, int& c) {
  using C = Tile32<T, D>;
  r = P / C::RCH;
  c = (P % C::RCH) ^ C::nkey(r);
}

// Physical chunk P of a column tile -> (row d, logical chunk)
template <typename T, int D>
__device__ __forceinline__ void col_chunk(int P, int& d, int& c) {
  using C = Tile32<T, D>;
  d = P / C::CCH;
  c = (P % C::CCH) ^ C::ckey(d);
}

// Fill NCHUNK 16-byte chunks of an LDS tile with direct global -> LDS loads;
// src(P) is the global address of the data for physical chunk P.  Completion
// is tracked by vmcnt: wait (lds_dma_wait) before the barrier that publishes
// the tile.
template <int NTH, int NCHUNK, typename SrcFn>
__device__ __forceinline__ void dma_tile(void* lds, SrcFn src, int tid) {
  const int w = tid >> 6, lane = tid & 63;
#pragma unroll
  for (int j = 0; j < (NCHUNK + NTH - 1) / NTH; ++j) {
    const int first = j * NTH + 64 * w;   // first physical chunk of this wave's load
    if (NCHUNK % NTH == 0 || first < NCHUNK)
      __builtin_amdgcn_global_load_lds(src(first + lane), (char*)lds + 16 * first, 16, 0, 0);
  }
}

// The 64-bit value whose 32-bit halves came back as int (readfirstlane
// returns int): each half is taken as uint32_t, so a low half with bit 31 set
// is zero-extended instead of sign-extended into the high half.
__host__ __device__ constexpr uint64_t u64_from_halves(int lo, int hi) {
  return ((uint64_t)(uint32_t)hi << 32) | (uint64_t)(uint32_t)lo;
}
static_assert(u64_from_halves((int)0x80001000u, 0x7ffe) == 0x00007ffe80001000ull,
              "a base address with bit 31 set must survive the split into halves");

// The rows of a tile's two queries tA and tB (tB < 0: none; its lanes then
// read tA's rows) as unsigned byte offsets from the lower of the two rows,
// t0: the DMA requests add them to unsigned per-lane offsets, so neither may
// be negative.  CSR entries ascend within a block, but a caller's CSR need
// not: a difference taken from tA alone would wrap to about 4 GB past the
// base when tB < tA.
struct PairRows {
  int t0;
  uint32_t dA, dB;
};
__host__ __device__ constexpr PairRows pair_rows(int tA, int tB, uint32_t row_bytes) {
  const int tb = tB >= 0 ? tB : tA;
  const int t0 = tA < tb ? tA : tb;
  return PairRows{t0, (uint32_t)(tA - t0) * row_bytes, (uint32_t)(tb - t0) * row_bytes};
}
static_assert(pair_rows(7, 3, 4096).t0 == 3 && pair_rows(7, 3, 4096).dA == 4 * 4096 &&
                  pair_rows(7, 3, 4096).dB == 0,
              "query B before query A: both offsets from B's row");
static_assert(pair_rows(3, 7, 256).t0 == 3 && pair_rows(3, 7, 256).dA == 0 && pair_rows(3, 7, 256).dB == 4 * 256,
              "ascending queries: from A's row");
static_assert(pair_rows(5, -1, 256).t0 == 5 && pair_rows(5, -1, 256).dB == 0, "no query B: A's row twice");

// Flat rows (groups of G < 16 heads): row R of a group is query R / G, head
// R % G, and a tile is rows R0 .. R0 + 31.  The queries that see key `key`
// form one run, so its rows are one run too:
//   window (window > 0): key <= t < key + window  <=>  key G <= R < (key + window) G
//   compression (window = 0): t >= key cd + cl - 1  <=>  R >= (key cd + cl - 1) G
// (t = floor(R / G) >= m  <=>  R >= m G, and t < m  <=>  R < m G).
// Returns bit r set for the tile rows r that see the key.
__host__ __device__ constexpr uint32_t flat_rows_seeing(int key, int R0, int G, int window, int cl, int cd) {
  int lo = window > 0 ? key * G - R0 : (key * cd + cl - 1) * G - R0;
  int hi = window > 0 ? (key + window) * G - R0 : 32;
  lo = lo < 0 ? 0 : (lo > 32 ? 32 : lo);
  hi = hi < 0 ? 0 : (hi > 32 ? 32 : hi);
  return lo < hi ? (uint32_t)(((1ull << hi) - 1ull) & ~((1ull << lo) - 1ull)) : 0u;
}
// Whether a flat tile needs the per-element test for the 32 keys kw ..
// kw + 31: false only when every one of them is seen by every row of the
// tile up to row rhi (the last present row).
__host__ __device__ constexpr bool flat_tile_needs_mask(int kw, int R0, int rhi, int G, int window, int cl,
                                                        int cd) {
  const int tf = R0 / G;                                 // the tile's first query
  const int tl = (R0 + 31 < rhi ? R0 + 31 : rhi) / G;    // and its last present one
  const int wlast = kw + 31;
  return window > 0 ? !(tf >= wlast && tl - window < kw) : !(wlast * cd + cl - 1 <= tf);
}
static_assert(flat_rows_seeing(5, 0, 6, 512, 0, 0) == ~((1u << 30) - 1u), "window: rows of queries >= 5");
static_assert(flat_rows_seeing(0, 0, 6, 3, 0, 0) == (1u << 18) - 1u, "window of 3: queries 0 .. 2");
static_assert(flat_rows_seeing(1, 270, 6, 0, 32, 16) == ~((1u << 12) - 1u),
              "compression, l 32 / d 16: key 1 seen by queries >= 47, rows >= 282");
static_assert(flat_rows_seeing(1, 60, 6, 0, 32, 16) == 0u, "compression: no row of queries 10 .. 15 sees key 1");

// Direct global -> LDS loads as volatile asm (lane i writes lds + SIZE i):
// the compiler neither tracks them nor adds waits for them, so LDS reads of
// other stages are not held behind loads still in flight.  The caller owns
// the ordering: vm_wait() before the barrier that publishes the data, and no
// reuse of a stage before the barrier that retires it.  `lds` must be
// wave-uniform; M0 is written here and is used by nothing else in the
// kernels that call these.
__device__ __forceinline__ uint32_t lds_addr_uniform(const void* lds) {
  // a generic pointer into LDS carries the LDS byte address in its low 32
  // bits (the aperture is the high half), so truncation is the conversion
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
}
__device__ __forceinline__ void lds_dma16(const void* gsrc, void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(lds_addr_uniform(lds)), "v"(gsrc) : "memory", "m0");
}
// As lds_dma16 with a wave-uniform 64-bit base and a per-lane 32-bit byte
// offset (the SGPR-base form: no per-lane 64-bit address arithmetic).
__device__ __forceinline__ void lds_dma16_sbase(const void* sbase, uint32_t voff, void* lds) {
  const uint64_t b = (uint64_t)(uintptr_t)sbase;
  const uint64_t bu = u64_from_halves(__builtin_amdgcn_readfirstlane((uint32_t)b),
                                      __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds_addr_uniform(lds)), "v"(voff), "s"(bu) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void* gsrc, void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :: "s"(lds_addr_uniform(lds)), "v"(gsrc) : "memory", "m0");
}

// As dma_tile, but through lds_dma16 and with every wave issuing the same
// number of loads (ceil(NCHUNK / NTH); surplus loads repeat a chunk of the
// tile with the same data), so a wave's outstanding-load count per tile is a
// constant that partial vmcnt waits can rely on.  NCHUNK must be a multiple
// of 64.
template <int NTH, int NCHUNK, typename SrcFn>
__device__ __forceinline__ void dma_tile_uniform(void* lds, SrcFn src, int tid) {
  static_assert(NCHUNK % 64 == 0, "tile chunks come in whole waves");
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
#pragma unroll
  for (int j = 0; j < (NCHUNK + NTH - 1) / NTH; ++j) {
    const int first = (j * NTH + 64 * w) % NCHUNK;
    lds_dma16(src(first + lane), (char*)lds + 16 * first);
  }
}
template <int NTH, int NCHUNK>
constexpr int dma_uniform_loads() { return (NCHUNK + NTH - 1) / NTH; }

// The source row a row-tile request starts from and the last tile row inside
// the source (nrows >= 1).  A tile that starts at or past the end (r0 >=
// nrows) reads row nrows - 1 for all its rows: with its start clamped, the
// per-lane clamp below subtracts at most a lane's own row, so no unsigned
// offset can wrap below the base.  Unclamped, such a tile's `last` was
// negative and the subtraction wrapped to about 4 GB past the base.
struct TileRows {
  int base, last;
};
__host__ __device__ constexpr TileRows tile_rows(int r0, int nrows) {
  const int b = r0 < nrows ? r0 : nrows - 1;
  return TileRows{b, nrows - 1 - b};
}
static_assert(tile_rows(96, 95).base == 94 && tile_rows(96, 95).last == 0, "a tile past the end reads the last row");
static_assert(tile_rows(64, 95).base == 64 && tile_rows(64, 95).last == 30, "a tile crossing the end");
static_assert(tile_rows(0, 95).last == 94, "a tile inside the source");

// dma_tile_uniform for [32][D] row tiles of a [rows][D] source, with the
// per-thread part of every address (row and chunk inside the tile) computed
// once by init: a request is a wave-uniform base plus constant per-lane
// offsets (lds_dma16_sbase), so it costs no per-lane address arithmetic.
// NAT: natural row order (nrow_chunk), else the permuted order of row_chunk.
// Rows at or past nrows repeat row nrows - 1.
template <typename T, int D, int NTH, bool NAT>
struct RowTileDma {
  using C = Tile32<T, D>;
  static constexpr int NL = dma_uniform_loads<NTH, C::ROW_CHUNKS>();
  int row[NL];
  uint32_t off[NL];
  __device__ __forceinline__ void init(int tid) {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int P = (j * NTH + 64 * w) % C::ROW_CHUNKS + lane;
      int r, c;
      if constexpr (NAT)
        nrow_chunk<T, D>(P, r, c);
      else
        row_chunk<T, D>(P, r, c);
      row[j] = r;
      off[j] = (uint32_t)((r * D + c * C::EPC) * (int)sizeof(T));
    }
  }
  // rows r0 .. r0 + 31 of src -> lds (nrows >= 1; a tile from r0 >= nrows
  // reads row nrows - 1 throughout)
  __device__ __forceinline__ void request(void* lds, const T* src, int r0, int nrows, int tid) const {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const TileRows tr = tile_rows(r0, nrows);
    const T* base = src + (int64_t)tr.base * D;
    const int last = tr.last;   // last row of the tile inside the source
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int first = (j * NTH + 64 * w) % C::ROW_CHUNKS;
      uint32_t o = off[j];
      if (last < 31 && row[j] > last) o -= (uint32_t)((row[j] - last) * D * (int)sizeof(T));
      lds_dma16_sbase(base, o, (char*)lds + 16 * first);
    }
  }
};

// The same for [D][32] column tiles of a transposed [D][Lp] source (keys kb ..
// kb + 31 of every row d; Lp covers every requested key, no clamping).
template <typename T, int D, int NTH>
struct ColTileDma {
  using C = Tile32<T, D>;
  static constexpr int NL = dma_uniform_loads<NTH, C::COL_CHUNKS>();
  uint32_t off[NL];
  __device__ __forceinline__ void init(int tid, int Lp) {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int P = (j * NTH + 64 * w) % C::COL_CHUNKS + lane;
      int d, c;
      col_chunk<T, D>(P, d, c);
      off[j] = (uint32_t)((d * Lp + c * C::EPC) * (int)sizeof(T));
    }
  }
  __device__ __forceinline__ void request(void* lds, const T* src, int kb, int tid) const {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int first = (j * NTH + 64 * w) % C::COL_CHUNKS;
      lds_dma16_sbase(src + kb, off[j], (char*)lds + 16 * first);
    }
  }
};

__device__ __forceinline__ void lds_dma_wait() { __builtin_amdgcn_s_waitcnt(0); }

// LDS written by some lanes of a wave and read by others: the writes are
// visible after this (a wave-scope fence and barrier).
__device__ __forceinline__ void wave_fence() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Wait for this wave's LDS operations only (lgkmcnt 0; vmcnt and expcnt at
// their maxima): a stage's reads are complete before a DMA refills it.
__device__ __forceinline__ void lds_reads_done() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order); LDS and export counters are not waited on.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Wait until at most BASE + min(n, K) * STEP vector-memory operations are
// outstanding; n is wave-uniform and picks one of K + 1 immediates.
template <int BASE, int STEP, int K>
__device__ __forceinline__ void vm_wait_steps(int n) {
  if constexpr (K == 0) {
    vm_wait<BASE>();
  } else {
    if (n >= K)
      vm_wait<BASE + K * STEP>();
    else
      vm_wait_steps<BASE, STEP, K - 1>(n);
  }
}

// Key-tile pipeline of the query-outer kernels: NST stages, tiles 0 ..
// NST-2 requested up front; iteration i waits for tile i (the NST-2 younger
// tiles stay in flight), passes the workgroup barrier -- after which no wave
// reads tile i-1 -- refills that stage with tile i + NST - 1 and computes
// tile i.  LT: vector-memory loads one wave issues per tile (the loop issues
// no other vector-memory operation).
template <int NST, int LT, typename Req, typename Body>
__device__ __forceinline__ void key_pipeline(int ntile, Req request, Body body) {
  static_assert(NST >= 2 && (NST - 1) * LT < 64, "in-flight operations exceed the vmcnt range");
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < ntile) request(p);
  for (int it = 0; it < ntile; ++it) {
    if (it + NST - 2 < ntile)
      vm_wait<(NST - 2) * LT>();
    else
      vm_wait<0>();
    __syncthreads();
    if (it + NST - 1 < ntile) request(it + NST - 1);
    body(it);
  }
}

// f(integral_constant<int, i>) for i = B .. E-1, unrolled at compile time
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// key_pipeline unrolled over its NST stages: request(i, st) and body(it, st)
// also receive the stage as a compile-time constant st (integral_constant),
// so that stage addresses are immediates rather than per-tile arithmetic.
template <int NST, int LT, typename Req, typename Body>
__device__ __forceinline__ void key_pipeline_st(int ntile, Req request, Body body) {
  static_assert(NST >= 2 && (NST - 1) * LT < 64, "in-flight operations exceed the vmcnt range");
  static_for<0, NST - 1>([&](auto p) {
    if (p.value < ntile) request(p.value, p);
  });
  for (int it0 = 0; it0 < ntile; it0 += NST) {
    static_for<0, NST>([&](auto p) {
      const int it = it0 + p.value;
      if (it >= ntile) return;
      if (it + NST - 2 < ntile)
        vm_wait<(NST - 2) * LT>();
      else
        vm_wait<0>();
      __syncthreads();
      if (it + NST - 1 < ntile) request(it + NST - 1, std::integral_constant<int, (p.value + NST - 1) % NST>{});
      body(it, p);
    });
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 8 consecutive elements of a row (one 16-byte load for bf16, two for float)
__device__ __forceinline__ void load8(const bf16* p, float (&x)[8]) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)v[i];
}
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = a[i], x[4 + i] = b[i];
}
__device__ __forceinline__ void store8(bf16* p, const float (&x)[8]) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)x[i];
  *reinterpret_cast<bf16x8*>(p) = v;
}
__device__ __forceinline__ void store8(float* p, const float (&x)[8]) {
  *reinterpret_cast<f32x4*>(p) = (f32x4){x[0], x[1], x[2], x[3]};
  *reinterpret_cast<f32x4*>(p + 4) = (f32x4){x[4], x[5], x[6], x[7]};
}
__device__ __forceinline__ void load8(const f16* p, float (&x)[8]) {
  const f16x8 v = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)v[i];
}
// store8 as a non-temporal store, for rows that consecutive lanes write whole
// (one 16-byte chunk each) and that a later launch reads: they need not stay
// cached.  Float rows take two stores a lane, each covering every other chunk
// of the row: those keep the cached store, so that the L2 merges the halves of
// a line before it goes to memory.
__device__ __forceinline__ void store8_nt(bf16* p, const float (&x)[8]) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (bf16)x[i];
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void store8_nt(float* p, const float (&x)[8]) { store8(p, x); }
// 16-bit rows of D >= 64 elements fill whole 128-byte lines; shorter rows
// share lines with rows that other instructions write, so they keep the cached
// store
template <int D> constexpr bool kWholeLines = D >= 64;
template <bool NT, typename T> __device__ __forceinline__ void store8_as(T* p, const float (&x)[8]) {
  if constexpr (NT)
    store8_nt(p, x);
  else
    store8(p, x);
}

// Stores 8 consecutive elements of a branch-output row and leaves in x the
// values as stored: rounded to TO, or for the NSA_F16S form (TO = f16) scaled
// by the row's power of two (f16s_row_scale), which the LPR consecutive lanes
// holding the row agree on through an xor reduction of their maxima; lane
// `first` of them writes it to *scale.
template <typename TO, int LPR, bool NT = false>
__device__ __forceinline__ void store_branch8(TO* p, float (&x)[8], float* scale, bool first) {
  if constexpr (IsF16<TO>::value) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
#pragma unroll
    for (int k = 1; k < LPR; k <<= 1) m = fmaxf(m, __shfl_xor(m, k, kWave));
    const float sc = f16s_row_scale(m), inv = 1.0f / sc;
    f16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] = (f16)(x[i] * inv);
      x[i] = (float)v[i] * sc;
    }
    if constexpr (NT)
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
    else
      *reinterpret_cast<f16x8*>(p) = v;
    if (first) *scale = sc;
  } else {
    if constexpr (NT)
      store8_nt(p, x);
    else
      store8(p, x);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = to_f32(from_f32<TO>(x[i]));
  }
}
// Loads 8 consecutive elements of a branch-output row as stored (the row's
// scale applied for the NSA_F16S form).
template <typename TO>
__device__ __forceinline__ void load_branch8(const TO* p, float (&x)[8], const float* scale) {
  load8(p, x);
  if constexpr (IsF16<TO>::value) {
    const float sc = *scale;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] *= sc;
  }
}

// 8 consecutive elements of a row as loaded (one 16-byte load for bf16, two
// for float), converted at use.  load_nt: a non-temporal load, for data read
// once (the selection partials), which then does not displace cached lines.
template <typename T> struct Raw8;
template <> struct Raw8<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ void load_nt(const bf16* p) {
    v = __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
  }
  __device__ __forceinline__ float get(int i) const { return (float)v[i]; }
  __device__ __forceinline__ void keep_if(bool ok) {   // zero, bit for bit, unless ok
    u32x4 u = __builtin_bit_cast(u32x4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = ok ? u[i] : 0u;
    v = __builtin_bit_cast(bf16x8, u);
  }
};
template <> struct Raw8<f16> {
  f16x8 v;
  __device__ __forceinline__ void load(const f16* p) { v = *reinterpret_cast<const f16x8*>(p); }
  __device__ __forceinline__ void load_nt(const f16* p) {
    v = __builtin_bit_cast(f16x8, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
  }
  __device__ __forceinline__ float get(int i) const { return (float)v[i]; }
  __device__ __forceinline__ void keep_if(bool ok) {   // zero, bit for bit, unless ok
    u32x4 u = __builtin_bit_cast(u32x4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = ok ? u[i] : 0u;
    v = __builtin_bit_cast(f16x8, u);
  }
};
template <> struct Raw8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ void load_nt(const float* p) {
    a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
  }
  __device__ __forceinline__ float get(int i) const { return i < 4 ? a[i] : b[i - 4]; }
  __device__ __forceinline__ void keep_if(bool ok) {
    u32x4 ua = __builtin_bit_cast(u32x4, a), ub = __builtin_bit_cast(u32x4, b);
#pragma unroll
    for (int i = 0; i < 4; ++i) ua[i] = ok ? ua[i] : 0u, ub[i] = ok ? ub[i] : 0u;
    a = __builtin_bit_cast(f32x4, ua);
    b = __builtin_bit_cast(f32x4, ub);
  }
};

}  // namespace nsa
