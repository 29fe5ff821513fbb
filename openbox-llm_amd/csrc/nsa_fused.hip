// The gated three-branch layer behind two C entry points (nsa_fused_fwd /
// nsa_fused_bwd): the launch sequence of the Python autograd boundary
// (nsa_hip_ops.fused_forward / fused_backward) for callers without Python.
// Host code only: every launch goes through the library's own entry points,
// in the same order and with the same arguments, so the results are the
// Python path's bit for bit.
//
// Two caller buffers, carved by the same plan on both calls:
//   ctx     -- written by the forward, read by the backward (what autograd
//              would save): pooled keys, packed q, the three branch outputs
//              (float32), their lse, the block -> query CSR;
//   scratch -- transient, any contents on entry: transposed K/V copies, the
//              selection partials of the forward, then the backward's row
//              statistics, float32 dK/dV accumulators, dQ partials and the
//              deterministic-merge partial rows.
#include <cstddef>
#include <cstdint>

#include "nsa_launch.h"
#include "nsa_items.h"

namespace {

constexpr int kFwdChunk = 128;    // CSR queries per selection forward work item
constexpr int kDkdvChunk = 512;   // CSR queries per selection dK/dV work item

struct Carver {
  size_t off = 0;
  char* base = nullptr;
  void* take(size_t bytes) {
    off = (off + 255) & ~(size_t)255;
    void* p = base ? base + off : nullptr;
    off += bytes;
    return p;
  }
};

struct Dims {
  int B, Hq, Hkv, T, D, l, d, ls, n_sel, window, force_init, n_local, dtype, pooled;
  int G() const { return Hq / Hkv; }
  int ncmp() const { return T >= l ? (T - l) / d + 1 : 0; }
  int S() const { const int n = T / ls; return n_sel < n ? n_sel : n; }
  int nblk() const { return (T + ls - 1) / ls; }
  size_t es() const { return dtype == NSA_BF16 ? 2 : 4; }
  int64_t rows() const { return (int64_t)B * Hq * T; }
  // the branch outputs kept for the backward: NSA_F16S for bf16 inputs,
  // float32 for float32 inputs (unrounded either way but for fp16's 11 bits)
  int o_dtype() const { return dtype == NSA_BF16 ? NSA_F16S : NSA_F32; }
  size_t o_bytes() const { return dtype == NSA_BF16 ? (size_t)rows() * (2 * D + 4) : (size_t)rows() * D * 4; }
  int64_t kv(int L) const { return (int64_t)B * Hkv * L * D; }
  bool ok() const {
    return B > 0 && Hkv > 0 && Hq % Hkv == 0 && (D == 16 || D == 32 || D == 64 || D == 128) && l >= 1 && d >= 1 &&
           ls >= 16 && ls % 16 == 0 && n_sel >= 1 && window >= 1 && n_local >= 0 && T >= l && T >= ls &&
           (dtype == NSA_F32 || dtype == NSA_BF16);
  }
};

// The state the forward leaves for the backward.
struct Ctx {
  void *k_cmp, *v_cmp, *qp;
  void *o_c, *o_s, *o_w;
  float *lse_c, *lse_s, *lse_w;
  int32_t *q_of_block, *offsets, *pair_bh, *count;
};

Ctx carve_ctx(const Dims& m, void* base, size_t* bytes) {
  Carver c;
  c.base = (char*)base;
  Ctx x{};
  const int n = m.ncmp();
  x.k_cmp = m.pooled ? nullptr : c.take(m.kv(n) * m.es());
  x.v_cmp = m.pooled ? nullptr : c.take(m.kv(n) * m.es());
  x.qp = c.take((size_t)m.rows() * m.D * m.es());
  void** outs[3] = {&x.o_c, &x.o_s, &x.o_w};
  for (void** o : outs) *o = c.take(m.o_bytes());
  x.lse_c = (float*)c.take(m.rows() * sizeof(float));
  x.lse_s = (float*)c.take(m.rows() * sizeof(float));
  x.lse_w = (float*)c.take(m.rows() * sizeof(float));
  const size_t cap = (size_t)m.B * m.Hkv * m.T * m.S();
  x.q_of_block = (int32_t*)c.take(cap * sizeof(int32_t));
  x.offsets = (int32_t*)c.take((size_t)m.B * m.Hkv * (m.nblk() + 1) * sizeof(int32_t));
  x.pair_bh = (int32_t*)c.take(cap * sizeof(int32_t));
  x.count = (int32_t*)c.take(sizeof(int32_t));
  *bytes = c.off;
  return x;
}

struct FwdScratch {
  void *vt_c, *csr_ws, *vt_s, *o_part, *sel_ws, *vt_w;
  float* ml_part;
  size_t csr_bytes, sel_bytes;
};

FwdScratch carve_fwd(const Dims& m, void* base, size_t* bytes) {
  Carver c;
  c.base = (char*)base;
  FwdScratch x{};
  const int n = m.ncmp(), S = m.S();
  const int ns = nsa_sel_partial_slots(S, m.ls);
  x.vt_c = c.take((size_t)m.B * m.Hkv * m.D * nsa_padded_len(n) * m.es());
  x.csr_bytes = nsa_csr_workspace(m.B, m.Hkv, m.T, S, m.nblk());
  x.csr_ws = c.take(x.csr_bytes);
  x.vt_s = c.take((size_t)m.B * m.Hkv * m.D * nsa_padded_len(m.T) * m.es());
  x.o_part = c.take((size_t)m.rows() * ns * m.D * m.es());
  x.ml_part = (float*)c.take((size_t)m.rows() * ns * 2 * sizeof(float));
  x.sel_bytes = nsa_sel_fwd_bo_workspace(m.B, m.Hkv, m.T, S, m.ls, kFwdChunk);
  x.sel_ws = c.take(x.sel_bytes);
  x.vt_w = c.take((size_t)m.B * m.Hkv * m.D * nsa_padded_len(m.T) * m.es());
  *bytes = c.off;
  return x;
}

struct BwdScratch {
  float *dot, *rs, *coff, *dks, *dvs, *dkw, *dvw, *dkp, *dvp, *sel_part, *cmp_part;
  void *dop, *kt_s, *dq_part, *sel_ws, *kt_w, *kt_c;
  size_t sel_bytes, sel_part_bytes, cmp_part_bytes;
};

BwdScratch carve_bwd(const Dims& m, void* base, size_t* bytes, hipStream_t s) {
  Carver c;
  c.base = (char*)base;
  BwdScratch x{};
  const int n = m.ncmp(), S = m.S();
  const int ns = nsa_sel_partial_slots(S, m.ls);
  const bool f32 = m.dtype == NSA_F32;   // float32 gradients go straight to the caller's outputs
  x.dot = (float*)c.take(3 * m.rows() * sizeof(float));
  x.rs = (float*)c.take(3 * m.rows() * sizeof(float));
  x.coff = (float*)c.take(3 * m.rows() * sizeof(float));
  x.dop = c.take((size_t)m.rows() * m.D * m.es());
  x.kt_s = c.take((size_t)m.B * m.Hkv * m.D * nsa_padded_len(m.T) * m.es());
  x.dks = f32 ? nullptr : (float*)c.take(m.kv(m.T) * sizeof(float));
  x.dvs = f32 ? nullptr : (float*)c.take(m.kv(m.T) * sizeof(float));
  x.dq_part = c.take((size_t)m.rows() * ns * m.D * m.es());
  x.sel_bytes = nsa_sel_dkdv_workspace(m.B, m.Hkv, m.T, S, m.ls, kDkdvChunk);
  x.sel_ws = c.take(x.sel_bytes);
  x.sel_part_bytes = nsa_sel_dkdv_partial_bytes(m.B, m.Hkv, m.T, S, m.D, m.ls, kDkdvChunk);
  x.sel_part = (float*)c.take(x.sel_part_bytes);
  x.kt_w = c.take((size_t)m.B * m.Hkv * m.D * nsa_padded_len(m.T) * m.es());
  x.dkw = f32 ? nullptr : (float*)c.take(m.kv(m.T) * sizeof(float));
  x.dvw = f32 ? nullptr : (float*)c.take(m.kv(m.T) * sizeof(float));
  x.dkp = (f32 && m.pooled) ? nullptr : (float*)c.take(m.kv(n) * sizeof(float));
  x.dvp = (f32 && m.pooled) ? nullptr : (float*)c.take(m.kv(n) * sizeof(float));
  x.cmp_part_bytes = nsa_range_dkdv_partial_bytes(NSA_MODE_COMPRESS, m.B, m.Hkv, m.T, n, m.D, m.l, m.d, s);
  x.cmp_part = (float*)c.take(x.cmp_part_bytes);
  x.kt_c = c.take((size_t)m.B * m.Hkv * m.D * nsa_padded_len(n) * m.es());
  *bytes = c.off;
  return x;
}

#define NSA_TRY(call)             \
  do {                            \
    const int rc_ = (call);       \
    if (rc_ != NSA_OK) return rc_; \
  } while (0)

}  // namespace

extern "C" {

size_t nsa_fused_ctx_bytes(int B, int Hq, int Hkv, int T, int D, int cmp_block, int cmp_stride, int sel_block,
                           int n_sel, int window, int pooled, int dtype) {
  const Dims m{B, Hq, Hkv, T, D, cmp_block, cmp_stride, sel_block, n_sel, window, 0, 0, dtype, pooled};
  if (!m.ok()) return 0;
  size_t bytes = 0;
  carve_ctx(m, nullptr, &bytes);
  return bytes;
}

size_t nsa_fused_scratch_bytes(int B, int Hq, int Hkv, int T, int D, int cmp_block, int cmp_stride, int sel_block,
                               int n_sel, int window, int pooled, int dtype, void* stream) {
  const Dims m{B, Hq, Hkv, T, D, cmp_block, cmp_stride, sel_block, n_sel, window, 0, 0, dtype, pooled};
  if (!m.ok()) return 0;
  size_t fb = 0, bb = 0;
  carve_fwd(m, nullptr, &fb);
  carve_bwd(m, nullptr, &bb, (hipStream_t)stream);
  return fb > bb ? fb : bb;
}

int nsa_fused_fwd(const void* q, const void* kc, const void* vc, const void* ks, const void* vs, const void* kw,
                  const void* vw, const void* gate, int32_t* block_idx, int idx_given, void* out, void* ctx,
                  size_t ctx_bytes, void* scratch, size_t scratch_bytes, int B, int Hq, int Hkv, int T, int D,
                  int cmp_block, int cmp_stride, int sel_block, int n_sel, int window, int force_init, int n_local,
                  int pooled, int dtype, void* stream) {
  const Dims m{B, Hq, Hkv, T, D, cmp_block, cmp_stride, sel_block, n_sel, window, force_init, n_local, dtype, pooled};
  NSA_CHECK(m.ok(), dtype == NSA_F32 || dtype == NSA_BF16 ? NSA_ERR_SHAPE : NSA_ERR_DTYPE);
  NSA_CHECK(q && kc && vc && ks && vs && kw && vw && gate && block_idx && out && ctx && scratch, NSA_ERR_ARG);
  hipStream_t s = (hipStream_t)stream;
  size_t cb = 0, sb = 0;
  carve_ctx(m, nullptr, &cb);
  NSA_CHECK(ctx_bytes >= cb, NSA_ERR_WORKSPACE);
  NSA_CHECK(scratch_bytes >= nsa_fused_scratch_bytes(B, Hq, Hkv, T, D, cmp_block, cmp_stride, sel_block, n_sel,
                                                     window, pooled, dtype, stream),
            NSA_ERR_WORKSPACE);
  const Ctx x = carve_ctx(m, ctx, &cb);
  const FwdScratch w = carve_fwd(m, scratch, &sb);
  const int n = m.ncmp(), S = m.S(), Lpn = nsa_padded_len(n), Lpt = nsa_padded_len(T);
  const void* k_cmp = pooled ? kc : x.k_cmp;
  const void* v_cmp = pooled ? vc : x.v_cmp;
  if (!pooled) {
    NSA_TRY(nsa_pool_fwd(kc, x.k_cmp, B, Hkv, T, D, cmp_block, cmp_stride, dtype, stream));
    NSA_TRY(nsa_pool_fwd(vc, x.v_cmp, B, Hkv, T, D, cmp_block, cmp_stride, dtype, stream));
  }
  // compression (its forward also writes the packed q of the selection kernels)
  NSA_TRY(nsa_transpose_kv(v_cmp, w.vt_c, B * Hkv, n, D, Lpn, dtype, stream));
  NSA_TRY(nsa_range_fwd(NSA_MODE_COMPRESS, q, k_cmp, w.vt_c, x.o_c, x.lse_c, B, Hq, Hkv, T, n, D, 0, cmp_block,
                        cmp_stride, x.qp, dtype, m.o_dtype(), stream));
  if (!idx_given)
    NSA_TRY(nsa_importance_topn(q, k_cmp, x.lse_c, block_idx, nullptr, B, Hq, Hkv, T, n, D, cmp_block, cmp_stride,
                                sel_block, n_sel, force_init, n_local, dtype, stream));
  // selection partials over the block -> query CSR
  NSA_TRY(nsa_csr_build(block_idx, x.q_of_block, x.offsets, x.pair_bh, x.count, w.csr_ws, w.csr_bytes, B, Hkv, T,
                        S, sel_block, m.nblk(), 1, stream));
  NSA_TRY(nsa_transpose_kv(vs, w.vt_s, B * Hkv, T, D, Lpt, dtype, stream));
  NSA_TRY(nsa_sel_fwd_bo(x.qp, ks, w.vt_s, x.q_of_block, x.offsets, w.o_part, w.ml_part, w.sel_ws, w.sel_bytes, B, Hq,
                         Hkv, T, D, S, sel_block, kFwdChunk, dtype, stream));
  // window, finishing the rows: selection merge and gate
  NSA_TRY(nsa_transpose_kv(vw, w.vt_w, B * Hkv, T, D, Lpt, dtype, stream));
  return nsa_range_fwd_finish(NSA_MODE_WINDOW, q, kw, w.vt_w, x.o_w, x.lse_w, B, Hq, Hkv, T, T, D, window, 1, 1,
                              w.o_part, w.ml_part, block_idx, S, sel_block, x.o_s, x.lse_s, x.o_c, gate, out, dtype,
                              m.o_dtype(), dtype, stream);
}

int nsa_fused_bwd(const void* dout, const void* q, const void* kc, const void* vc, const void* ks, const void* vs,
                  const void* kw, const void* vw, const void* gate, const int32_t* block_idx, const void* ctx,
                  size_t ctx_bytes, void* scratch, size_t scratch_bytes, void* dq, void* dkc, void* dvc, void* dks,
                  void* dvs, void* dkw, void* dvw, void* dgate, int B, int Hq, int Hkv, int T, int D, int cmp_block,
                  int cmp_stride, int sel_block, int n_sel, int window, int pooled, int dtype, void* stream) {
  const Dims m{B, Hq, Hkv, T, D, cmp_block, cmp_stride, sel_block, n_sel, window, 0, 0, dtype, pooled};
  NSA_CHECK(m.ok(), dtype == NSA_F32 || dtype == NSA_BF16 ? NSA_ERR_SHAPE : NSA_ERR_DTYPE);
  NSA_CHECK(dout && q && ks && vs && kw && vw && gate && block_idx && ctx && scratch, NSA_ERR_ARG);
  NSA_CHECK(dq && dkc && dvc && dks && dvs && dkw && dvw && dgate && (!pooled || (kc && vc)), NSA_ERR_ARG);
  hipStream_t s = (hipStream_t)stream;
  size_t cb = 0, sb = 0;
  carve_ctx(m, nullptr, &cb);
  NSA_CHECK(ctx_bytes >= cb, NSA_ERR_WORKSPACE);
  NSA_CHECK(scratch_bytes >= nsa_fused_scratch_bytes(B, Hq, Hkv, T, D, cmp_block, cmp_stride, sel_block, n_sel,
                                                     window, pooled, dtype, stream),
            NSA_ERR_WORKSPACE);
  const Ctx x = carve_ctx(m, (void*)ctx, &cb);
  const BwdScratch w = carve_bwd(m, scratch, &sb, s);
  const int n = m.ncmp(), S = m.S(), G = m.G(), Lpn = nsa_padded_len(n), Lpt = nsa_padded_len(T);
  const int64_t R = m.rows();
  const bool f32 = dtype == NSA_F32;
  const void* k_cmp = pooled ? kc : x.k_cmp;
  const void* v_cmp = pooled ? vc : x.v_cmp;
  float* dks32 = f32 ? (float*)dks : w.dks;
  float* dvs32 = f32 ? (float*)dvs : w.dvs;
  float* dkw32 = f32 ? (float*)dkw : w.dkw;
  float* dvw32 = f32 ? (float*)dvw : w.dvw;
  float* dkp32 = (f32 && pooled) ? (float*)dkc : w.dkp;
  float* dvp32 = (f32 && pooled) ? (float*)dvc : w.dvp;
  // gate backward, row dots of the three branches, dO packed for the selection
  NSA_TRY(nsa_bwd_prep(dout, x.o_c, x.o_s, x.o_w, gate, dgate, x.lse_c, x.lse_s, x.lse_w, w.dot, w.rs, w.coff,
                       w.dop, G, T, R, D, 3, dtype, m.o_dtype(), dtype, stream));
  // selection dK/dV and dQ partials (block-outer, deterministic merge)
  NSA_TRY(nsa_transpose_kv(ks, w.kt_s, B * Hkv, T, D, Lpt, dtype, stream));
  NSA_TRY(nsa_sel_dkdv(x.qp, ks, vs, w.kt_s, w.dop, w.coff + R, w.dot + R, x.q_of_block, 1, x.offsets, x.count,
                       dks32, dvs32, w.sel_part, w.sel_part_bytes, w.dq_part, w.sel_ws, w.sel_bytes, B, Hq, Hkv, T, D,
                       S, sel_block, kDkdvChunk, dtype, stream));
  // window and compression dK/dV
  NSA_TRY(nsa_transpose_kv(kw, w.kt_w, B * Hkv, T, D, Lpt, dtype, stream));
  NSA_TRY(nsa_range_dkdv(NSA_MODE_WINDOW, q, kw, vw, dout, w.coff + 2 * R, w.dot + 2 * R, dkw32, dvw32, nullptr, 0, B,
                         Hq, Hkv, T, T, D, window, 1, 1, dtype, stream));
  NSA_TRY(nsa_range_dkdv(NSA_MODE_COMPRESS, q, k_cmp, v_cmp, dout, w.coff, w.dot, dkp32, dvp32, w.cmp_part,
                         w.cmp_part_bytes, B, Hq, Hkv, T, n, D, 0, cmp_block, cmp_stride, dtype, stream));
  // compression + window dQ in one launch, rows finished with the selection partials
  NSA_TRY(nsa_transpose_kv(k_cmp, w.kt_c, B * Hkv, n, D, Lpn, dtype, stream));
  NSA_TRY(nsa_range_dq_cw(q, dout, k_cmp, v_cmp, w.kt_c, x.lse_c, w.dot, w.rs, n, cmp_block, cmp_stride, kw, vw,
                          w.kt_w, x.lse_w, w.dot + 2 * R, w.rs + 2 * R, window, B, Hq, Hkv, T, D, w.dq_part, block_idx,
                          S, sel_block, dq, dtype, dtype, stream));
  // the key / value gradients in the input dtype
  if (!pooled) {
    NSA_TRY(nsa_pool_bwd(dkp32, NSA_F32, dkc, B, Hkv, T, D, cmp_block, cmp_stride, dtype, stream));
    NSA_TRY(nsa_pool_bwd(dvp32, NSA_F32, dvc, B, Hkv, T, D, cmp_block, cmp_stride, dtype, stream));
  } else if (!f32) {
    NSA_TRY(nsa_cast_f32(dkp32, dkc, m.kv(n), dtype, stream));
    NSA_TRY(nsa_cast_f32(dvp32, dvc, m.kv(n), dtype, stream));
  }
  if (!f32) {
    NSA_TRY(nsa_cast_f32(dks32, dks, m.kv(T), dtype, stream));
    NSA_TRY(nsa_cast_f32(dvs32, dvs, m.kv(T), dtype, stream));
    NSA_TRY(nsa_cast_f32(dkw32, dkw, m.kv(T), dtype, stream));
    NSA_TRY(nsa_cast_f32(dvw32, dvw, m.kv(T), dtype, stream));
  }
  return NSA_OK;
}

}  // extern "C"
