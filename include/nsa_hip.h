/* C-ABI of the MI355X (gfx950) Native Sparse Attention library, libnsa_hip.so.
 *
 * Plain pointers and sizes only.  Tensors are dense row-major:
 *   q, o, dO, dq      [B][Hq][T][D]
 *   k, v, dk, dv      [B][Hkv][Lk][D]      (Lk = T, or the pooled length)
 *   lse, dot, scale   [B][Hq][T]  float32
 *   block_idx         [B][Hkv][T][S] int32, -1 = empty slot
 *   gate logits       [B][Hq][T][3]
 * with query head h reading KV head h / (Hq / Hkv).  dtype is NSA_F32 or
 * NSA_BF16 for every tensor of the call not marked float.  Every launch goes
 * to `stream` (a hipStream_t); nothing is allocated and nothing synchronises
 * with the host.  Scratch memory is passed in by the caller (one entry point,
 * nsa_sel_dkdv_noalloc, uses a fixed device array of the library instead).
 *
 * Return value: NSA_OK (0) or a negative NSA_ERR_* code.  Host wrappers map
 * NSA_ERR_SHAPE / NSA_ERR_DTYPE to the reference's assertion failures
 * (nsa_selection_kernel.py:186-189) and the rest to runtime errors.
 *
 * Each entry point names the reference Python function whose work it takes
 * over (paths relative to the openbox-llm checkout).
 */
#ifndef NSA_HIP_H
#define NSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSA_OK 0
#define NSA_ERR_SHAPE -1
#define NSA_ERR_DTYPE -2
#define NSA_ERR_ARG -3
#define NSA_ERR_LAUNCH -4
#define NSA_ERR_WORKSPACE -5

#define NSA_F32 0
#define NSA_BF16 1
/* Only for the branch outputs a forward keeps for its backward (the o_dtype
 * of nsa_range_fwd, nsa_range_fwd_finish and nsa_bwd_prep, with bf16
 * inputs): fp16 rows [B][Hq][T][D], each stored divided by a power-of-two
 * scale s_r (1 unless the row's largest magnitude reaches 2^15), followed in
 * the same buffer by the float32 scales s_r [B][Hq][T].  Buffer bytes:
 * B*Hq*T*(2*D + 4).  Eight times finer than bf16 at half float32's size. */
#define NSA_F16S 2

#define NSA_MODE_WINDOW 0
#define NSA_MODE_COMPRESS 1

/* Library version (major * 100 + minor). */
int nsa_version(void);

/* Length of a transposed K/V copy row: Lk rounded up with >= 32 keys of zero
 * padding.  Transposed copies are [B*Hkv][D][nsa_padded_len(Lk)]. */
int nsa_padded_len(int Lk);

/* ---- layout helpers -------------------------------------------------------
 * x [BH][L][D] -> xt [BH][D][Lp] (Lp >= L, zero padded).  Used for the V^T /
 * K^T operands of the attention kernels. */
int nsa_transpose_kv(const void* x, void* xt, int BH, int L, int D, int Lp, int dtype, void* stream);

/* ---- compression pooling ---------------------------------------------------
 * Replaces block_mean_pool (nsa_fused_kernel.py:549-554): out[i] = mean of
 * x[i*d .. i*d+l-1]; n = (T-l)/d + 1 pooled tokens (T//l when l == d). */
int nsa_pool_fwd(const void* x, void* out, int B, int H, int T, int D, int l, int d, int dtype,
                 void* stream);
/* Gradient of nsa_pool_fwd.  dpool [B][H][n][D] in dpool_dtype; dx written. */
int nsa_pool_bwd(const void* dpool, int dpool_dtype, void* dx, int B, int H, int T, int D, int l, int d,
                 int dtype, void* stream);

/* Learned weighted pool over the same overlapping spans: the arithmetic of
 * BlockCompressor's pooling (nsa_model.py:100-123, before its projection),
 * sum_p w[p] (x[i*d + p] + P[p]), taken as sum_p w[p] x[i*d + p] + cvec with
 * cvec = w^T P.  w: the l softmax weights, float32; out [B][H][n][D] float32.
 * D % 8 == 0; x and out 16-byte aligned. */
int nsa_wpool_fwd(const void* x, const float* w, const float* cvec, float* out, int B, int H, int T, int D, int l,
                  int d, int dtype, void* stream);
/* Its gradient for x: dx[t] = sum over the spans i holding t of
 * w[t - i*d] dpool[i] (dpool float32 [B][H][n][D]); dx in dtype. */
int nsa_wpool_bwd(const float* dpool, const float* w, void* dx, int B, int H, int T, int D, int l, int d, int dtype,
                  void* stream);
/* Its gradient for the weights (the x part), per (b, h): dw_part[p][b*H + h] =
 * sum over (i, c) of x[b][h][i*d + p][c] dpool[b][h][i][c], float32 [l][B*H],
 * each summed in a fixed order; dw[p] is the sum of row p (the caller's, so
 * the library needs no scratch).  D % 8 == 0, D <= 2048, B*H < 65536. */
int nsa_wpool_dw(const void* x, const float* dpool, float* dw_part, int B, int H, int T, int D, int l, int d,
                 int dtype, void* stream);

/* ---- head split of the stacked projection -----------------------------------
 * Replaces the model's per-branch `_split_heads(proj(x)).contiguous()`
 * (nsa_model.py:192-194, 325-335), and the rotary embedding of a RoPE model,
 * for all branches in one pass.  y [B][T][W] is the row-major output of the
 * stacked projection; its columns hold nseg segments in order from column 0,
 * segment k being heads[k] heads of head_dim[k] channels (nseg <= 8); columns
 * past sum heads*head_dim <= W are padding (a pitch W % 8 == 0 lets 16-byte
 * pieces of every aligned segment move in one access).
 * outs[k] [B][heads[k]][T][head_dim[k]] gets segment k plus biases[k][h*hd+j]
 * (float32, or null; biases itself may be null), rotated when rotate[k] by the
 * half-split rotary with cos_t, sin_t float32 [T][hd/2] (all rotated segments
 * share one hd).  float32 arithmetic, one rounding per output; y and outs in
 * dtype. */
int nsa_heads_split(const void* y, void* const* outs, const float* const* biases, const int* heads,
                    const int* head_dim, const int* rotate, int nseg, const float* cos_t, const float* sin_t, int B,
                    int T, int W, int dtype, void* stream);
/* Gradient of nsa_heads_split for y: dy [B][T][W] from the outputs' gradients
 * douts[k] (same layout as outs[k]; a null entry is a zero gradient), the
 * inverse rotation applied to rotated segments, zeros in the padding columns.
 * Bias gradients are the caller's (sums over B and T). */
int nsa_heads_merge_grad(const void* const* douts, void* dy, const int* heads, const int* head_dim,
                         const int* rotate, int nseg, const float* cos_t, const float* sin_t, int B, int T, int W,
                         int dtype, void* stream);

/* ---- gate ------------------------------------------------------------------
 * Replaces the gate blend of nsa_fused_forward (nsa_fused_kernel.py:572-573):
 * out = sigmoid(g0) o_cmp + sigmoid(g1) o_slc + sigmoid(g2) o_win. rows = B*Hq*T. */
int nsa_gate_fwd(const void* gate, const void* o_cmp, const void* o_slc, const void* o_win, void* out,
                 int64_t rows, int D, int dtype, void* stream);

/* Backward prep.  o0 / o1 / o2 are in o_dtype: dtype, NSA_F32 when the
 * forward kept the branch outputs unrounded, or NSA_F16S (bf16 inputs) when
 * it kept them as scaled fp16 rows (nsa_range_fwd's o_dtype).
 * nbr == 1: dot[r] = dO[r] . o0[r] (the delta of
 * nsa_selection_backward.py:168).  nbr == 3: for each branch c,
 * dot[c*rows + r] = dO . o_c, rowscale[c*rows + r] = sigmoid(g_c) and
 * dgate[r][c] = sigmoid'(g_c) dot (autograd of nsa_fused_kernel.py:572-573).
 * coff (nullable, laid out like dot) receives the per-row exponent offset
 * lse_c[r] * log2(e) - log2(rowscale) (rowscale 1 when nbr == 1) that the
 * dK/dV kernels take; it needs lse_c for every branch c < nbr.  dout_packed
 * (nullable) receives dO in the nsa_pack_heads layout, G heads per KV head
 * and T queries per row block (rows = B Hq T); the selection branch's dot,
 * rowscale and coff (nbr == 1: the only branch, nbr == 3: branch 1) are then
 * written in the same packed row order [B][Hkv][T][G], the layout
 * nsa_sel_dkdv reads.  dgate_dtype: dtype, or NSA_F32 for dgate unrounded. */
int nsa_bwd_prep(const void* dout, const void* o0, const void* o1, const void* o2, const void* gate,
                 void* dgate, const float* lse0, const float* lse1, const float* lse2, float* dot,
                 float* rowscale, float* coff, void* dout_packed, int G, int T, int64_t rows, int D, int nbr,
                 int dtype, int o_dtype, int dgate_dtype, void* stream);

/* float32 accumulator -> dtype. */
int nsa_cast_f32(const float* x, void* y, int64_t n, int dtype, void* stream);

/* [B][Hkv*G][T][D] -> [B][Hkv][T][G][D]: the query-side layout the selection
 * kernels read (the G heads of one query and KV head contiguous).  No
 * reference counterpart: the reference reads [B][H][T][D] directly
 * (nsa_selection_kernel.py:186-189).  D * sizeof(dtype) must be 16 bytes
 * times a power of two; src and dst must not overlap. */
int nsa_pack_heads(const void* src, void* dst, int B, int Hkv, int G, int T, int D, int dtype, void* stream);

/* ---- selection branch ------------------------------------------------------
 * Forward: replaces _selection_fwd_kernel / selection_forward_triton
 * (nsa_selection_kernel.py:104-213, FSA variant :232-365).  vt is the
 * transposed copy of v from nsa_transpose_kv (Lp = nsa_padded_len(T)).
 * Writes o (dtype) and lse (float, -1e9 on rows with no visible key). */
int nsa_sel_fwd(const void* q, const void* k, const void* vt, const int32_t* block_idx, void* o,
                float* lse, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int dtype,
                void* stream);

/* Backward dQ (query-side half of _selection_bwd_kernel,
 * nsa_selection_backward.py:63-153).  kt = transposed k.  dot = dO . o per
 * row; rowscale (nullable) multiplies P per row (gate weight).  dq is float32:
 * dq = (accumulate ? dq : 0) + dQ. */
int nsa_sel_dq(const void* q, const void* k, const void* v, const void* kt, const void* dout,
               const int32_t* block_idx, const float* lse, const float* dot, const float* rowscale,
               float* dq, int accumulate, int B, int Hq, int Hkv, int T, int D, int S, int block_size,
               int dtype, void* stream);

/* Block -> query CSR (replaces build_block_to_query_csr, nsa_fsa.py:14-64):
 * pairs (t, j) with 0 <= j < n_blk and j*block_size <= t, grouped by (b, hkv, j),
 * query ascending.  n_blk is the reference's T / block_size (nsa_fsa.py:36) or
 * ceil(T / block_size) to include the trailing partial block.  Outputs:
 * q_of_block [cap] (the query t, or (t << b) | s with b = ceil(log2 S) -- s the pair's slot in block_idx --
 * when pack_slot != 0), block_offsets [B][Hkv][n_blk+1] (global offsets),
 * pair_bh [cap] (nullable), *pair_count (device int); entries past
 * *pair_count are unspecified.  cap = B*Hkv*T*S.  Pairs of one (b, hkv, j)
 * keep the input order ((t, slot) ascending, a block held twice by a row
 * twice).  Deterministic.  Scratch from nsa_csr_workspace. */
size_t nsa_csr_workspace(int B, int Hkv, int T, int S, int n_blk);
int nsa_csr_build(const int32_t* block_idx, int32_t* q_of_block, int32_t* block_offsets, int32_t* pair_bh,
                  int32_t* pair_count, void* workspace, size_t workspace_bytes, int B, int Hkv, int T, int S,
                  int block_size, int n_blk, int pack_slot, void* stream);

/* Backward dK/dV (block-outer; replaces _selection_dkdv_kernel /
 * selection_backward_fsa, nsa_selection_backward.py:207-334).  Consumes the
 * CSR above built with n_blk = ceil(T / block_size) (so a selected trailing
 * partial block, which the forward attends to, gets its gradient), split into
 * work items of at most `chunk` (<= 1024) queries; q_of_block holds (t << b) | s
 * when `packed`.  The entries of a block may come in any order (one per
 * (query, slot) pair of that block): nsa_csr_build writes them ascending,
 * another producer need not.  q and dout are in the nsa_pack_heads layout
 * [B][Hkv][T][G][D]; coff / dot, the row offsets and deltas of nsa_bwd_prep,
 * in the same packed row order [B][Hkv][T][G] (nsa_bwd_prep with
 * dout_packed writes them so), kt the
 * nsa_transpose_kv copy of k.  dk/dv: float32 [B][Hkv][T][D], every key
 * written.  dkdv_part (nullable, part_bytes >= nsa_sel_dkdv_partial_bytes):
 * each work item writes its dK/dV rows there and one more launch sums a
 * block's items in item order, so dk/dv are bit-identical run to run, as
 * the reference's disjoint per-block writes are
 * (nsa_selection_backward.py:207-275); without it the items merge with
 * float atomics into zero-filled dk/dv and the last bits may differ run to
 * run.  dq_part (nullable; needs packed and kt): the dQ of every (query,
 * slot, pass), scaled, in the input dtype,
 * [B][Hkv][T][nsa_sel_partial_slots(S, block_size)][G][D] -- summed by
 * nsa_sel_dq_reduce. */
size_t nsa_sel_dkdv_workspace(int B, int Hkv, int T, int S, int block_size, int chunk);
size_t nsa_sel_dkdv_partial_bytes(int B, int Hkv, int T, int S, int D, int block_size, int chunk);
int nsa_sel_dkdv(const void* q, const void* k, const void* v, const void* kt, const void* dout, const float* coff,
                 const float* dot, const int32_t* q_of_block, int packed, const int32_t* block_offsets, const int32_t* pair_count,
                 float* dk, float* dv, float* dkdv_part, size_t part_bytes, void* dq_part, void* workspace,
                 size_t workspace_bytes, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                 int dtype, void* stream);

/* nsa_sel_dkdv without a workspace argument: allocates nothing (no
 * hipMalloc, no allocating library call).  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  The
 * work-item list and counters live in a device array of the library,
 * NSA_SEL_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call
 * whose nsa_sel_dkdv_workspace(...) exceeds it returns NSA_ERR_WORKSPACE
 * before touching the device (about 65k work items: c3 needs 4.1k).  Every
 * call uses the array of its stream's device (the null stream: the current
 * device), which keeps the last call's contents (the call re-initialises what it reads): calls that overlap on
 * one GPU (two streams, two host threads) race and must be serialised by the
 * caller.  Arguments otherwise as nsa_sel_dkdv. */
#define NSA_SEL_NOALLOC_SCRATCH_BYTES ((size_t)1 << 20)
int nsa_sel_dkdv_noalloc(const void* q, const void* k, const void* v, const void* kt, const void* dout,
                         const float* coff, const float* dot, const int32_t* q_of_block, int packed,
                         const int32_t* block_offsets, const int32_t* pair_count, float* dk, float* dv,
                         void* dq_part, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                         int dtype, void* stream);

/* ---- block-outer selection forward and the partial merges ----------------
 * The FSA forward (replaces _selection_fwd_blockouter_kernel /
 * selection_forward_fsa, nsa_selection_kernel.py:232-365): work items as in
 * nsa_sel_dkdv over a CSR built with pack_slot (its entries in any order
 * within a block); for every (query, slot, pass)
 * it writes the unnormalised block-local output O_j = sum_k p_k v_k
 * (p_k = exp2(s_k - m_j)) to o_part and (m_j [log2 units], l_j = sum_k
 * p_k) float pairs to ml_part, as the reference's per-pair partials
 * (nsa_selection_kernel.py:286-290), both laid out
 * [B][Hkv][T][nsa_sel_partial_slots(S, block_size)][G] (x D for o_part).
 * q is in the nsa_pack_heads layout [B][Hkv][T][G][D], vt is the
 * nsa_transpose_kv copy of v; chunk <= 1024.  Workspace from
 * nsa_sel_fwd_bo_workspace.  o_part's elements are float32 for NSA_F32
 * inputs and fp16 for NSA_BF16 inputs (11 significant bits; the merged
 * output, and the backward's row dot dO . o through it, inherit the
 * partials' rounding): the partials of one block and 64-key pass are stored
 * divided by a power of two s, with m_j + log2 s and l_j / s, which merge to
 * the same output; s is 1 unless 64 max|v| over the pass's keys (a bound on
 * every such partial) reaches 2^15.  nsa_sel_merge and nsa_range_fwd_finish read them
 * with the inputs' dtype. */
int nsa_sel_partial_slots(int S, int block_size);
size_t nsa_sel_fwd_bo_workspace(int B, int Hkv, int T, int S, int block_size, int chunk);
int nsa_sel_fwd_bo(const void* q, const void* k, const void* vt, const int32_t* q_of_block,
                   const int32_t* block_offsets, void* o_part, float* ml_part, void* workspace,
                   size_t workspace_bytes, int B, int Hq, int Hkv, int T, int D, int S, int block_size, int chunk,
                   int dtype, void* stream);

/* Merge of the forward partials (the log-sum-exp combine of
 * nsa_selection_kernel.py:336-364): o and lse per row over the valid slots of
 * block_idx; rows with none get o = 0 and lse = -1e9.  dtype: the inputs'
 * of nsa_sel_fwd_bo (its partials fp16 for NSA_BF16); o in o_dtype: dtype,
 * or NSA_F32 unrounded. */
int nsa_sel_merge(const int32_t* block_idx, const void* o_part, const float* ml_part, void* o, float* lse, int B,
                  int Hq, int Hkv, int T, int D, int S, int block_size, int dtype, int o_dtype, void* stream);

/* dq_out = dq_acc (float32, nullable) + sum of the dQ partials of the valid
 * slots, written in the input dtype (the dQ reduce of
 * nsa_selection_backward.py:322-334).  dtype is the partials' and dq_out's
 * element type: the partial buffer is read as that type, so a code that
 * differs from the buffer's reads another size (a float32 code on a bf16
 * buffer reads past its end). */
int nsa_sel_dq_reduce(const int32_t* block_idx, const void* dq_part, const float* dq_acc, void* dq_out, int B,
                      int Hq, int Hkv, int T, int D, int S, int block_size, int dtype, void* stream);

/* ---- range branches (window / compression) ---------------------------------
 * Forward: replaces _range_attn_fwd_kernel / _range_attn_fwd_qtiled_kernel
 * (nsa_fused_kernel.py:61-119, 226-307).  mode NSA_MODE_WINDOW: key p visible
 * to t iff t-window < p <= t; NSA_MODE_COMPRESS: pooled token i visible iff
 * i*cmp_stride + cmp_block - 1 <= t.  k [B][Hkv][Lk][D], vt transposed v with
 * Lp = nsa_padded_len(Lk).  Writes o and lse; q_packed (nullable) also
 * receives q in the nsa_pack_heads layout (the rows are loaded anyway).
 * o_dtype: the type of o -- dtype (the reference's convention), NSA_F32 so
 * that a backward's row dots dO . o see the unrounded output, or NSA_F16S
 * (bf16 inputs; o then has B*Hq*T*(2*D + 4) bytes) for 11 significant bits
 * at half float32's size -- the fused layer keeps its branch outputs this
 * way for bf16 inputs, float32 for float32 inputs; only their gated sum is
 * returned. */
int nsa_range_fwd(int mode, const void* q, const void* k, const void* vt, void* o, float* lse, int B, int Hq,
                  int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride, void* q_packed, int dtype,
                  int o_dtype, void* stream);

/* nsa_range_fwd that also finishes the rows of the gated three-branch layer
 * (no reference counterpart as one call: nsa_sel_merge and nsa_gate_fwd
 * folded into the last branch's forward).  Besides this branch's o / lse it
 * merges the selection partials of nsa_sel_fwd_bo (o_part, ml_part, with the
 * [B][Hkv][T][S] block_idx of block size sel_block) into o_sel / lse_sel
 * and writes out = sigmoid(g0) o_cmp + sigmoid(g1) o_sel + sigmoid(g2) o from
 * the gate logits [B][Hq][T][3] (out in out_dtype: dtype, or NSA_F32
 * unrounded).  o, o_sel and o_cmp are in o_dtype (dtype, NSA_F32
 * unrounded, or NSA_F16S with bf16 inputs); the blend uses each branch as
 * stored. */
int nsa_range_fwd_finish(int mode, const void* q, const void* k, const void* vt, void* o, float* lse, int B,
                         int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride,
                         const void* o_part, const float* ml_part, const int32_t* block_idx, int S, int sel_block,
                         void* o_sel, float* lse_sel, const void* o_cmp, const void* gate, void* out, int dtype,
                         int o_dtype, int out_dtype, void* stream);

/* Backward dQ of the range branches (query-side half of
 * _range_attn_bwd_qtiled_kernel, nsa_fused_kernel.py:321-426): dq (float32)
 * receives this branch's dQ, added to its contents when `accumulate`.
 * With sel_part (nullable) the call instead finishes the rows and writes
 * dq_out in dq_out_dtype (dtype, or NSA_F32 unrounded): dq_out = (dq if
 * accumulate) + this branch's dQ +
 * the selection dQ partials of nsa_sel_dkdv for the valid slots of sel_idx
 * ([B][Hkv][T][S] block indices of block size sel_block) -- the role of
 * nsa_sel_dq_reduce folded into this kernel; dq is then only read. */
int nsa_range_dq(int mode, const void* q, const void* k, const void* v, const void* kt, const void* dout,
                 const float* lse, const float* dot, const float* rowscale, float* dq, int accumulate, int B,
                 int Hq, int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride,
                 const void* sel_part, const int32_t* sel_idx, int S, int sel_block, void* dq_out, int dtype,
                 int dq_out_dtype, void* stream);

/* Backward dQ of the compression and window branches in one launch, rows
 * finished with the selection dQ partials: equal to nsa_range_dq(window,
 * accumulate = 0) followed by nsa_range_dq(compression, accumulate = 1,
 * sel_part), without the float32 dQ buffer between them.  The compression
 * branch takes Lk pooled tokens (kc, vc, ktc), the window branch keys of the
 * query length (kw, vw, ktw); lse / dot / rowscale per branch as in
 * nsa_range_dq.  No counterpart in the reference (its two launches are
 * _range_attn_bwd_qtiled_kernel, nsa_fused_kernel.py:321-426, once per
 * branch); sel_part, sel_idx and dq_out (in dq_out_dtype) are required. */
int nsa_range_dq_cw(const void* q, const void* dout, const void* kc, const void* vc, const void* ktc,
                    const float* lse_c, const float* dot_c, const float* rowscale_c, int Lk, int cmp_block,
                    int cmp_stride, const void* kw, const void* vw, const void* ktw, const float* lse_w,
                    const float* dot_w, const float* rowscale_w, int window, int B, int Hq, int Hkv, int T, int D,
                    const void* sel_part, const int32_t* sel_idx, int S, int sel_block, void* dq_out, int dtype,
                    int dq_out_dtype, void* stream);

/* Backward dK/dV of the range branches (key-outer; the key-side half of
 * _range_attn_bwd_qtiled_kernel).  coff / dot: row offsets and deltas from
 * nsa_bwd_prep.  dk/dv float32 [B][Hkv][Lk][D], every key written.  The
 * window has one writer per key.  Compression splits each key's queries into
 * chunks: with dkdv_part (nullable, part_bytes >=
 * nsa_range_dkdv_partial_bytes for the same stream's device) the chunks write
 * partial rows that one more launch sums in chunk order (bit-identical run
 * to run); without it they merge with float atomics into zero-filled dk/dv. */
size_t nsa_range_dkdv_partial_bytes(int mode, int B, int Hkv, int T, int Lk, int D, int cmp_block, int cmp_stride,
                                    void* stream);
int nsa_range_dkdv(int mode, const void* q, const void* k, const void* v, const void* dout, const float* coff,
                   const float* dot, float* dk, float* dv, float* dkdv_part, size_t part_bytes, int B, int Hq,
                   int Hkv, int T, int Lk, int D, int window, int cmp_block, int cmp_stride, int dtype, void* stream);

/* ---- the gated three-branch layer in two calls -------------------------------
 * nsa_fused_fwd / nsa_fused_bwd replace nsa_fused_forward and its autograd
 * (nsa_fused_kernel.py:560-573; with block_idx chosen here, the pooling /
 * importance / top-n of NSAAttention._forward_fused, nsa_model.py:306-370)
 * for callers without Python: every launch of the layer, in the order and
 * with the arguments of the Python boundary (bit-identical results).
 * q [B][Hq][T][D]; kc, vc [B][Hkv][T][D] (pooled = 0: mean-pooled here over
 * spans [i d, i d + l)) or the pooled tokens [B][Hkv][(T - l) / d + 1][D]
 * (pooled = 1: a learned compressor's output); ks, vs, kw, vw [B][Hkv][T][D];
 * gate logits [B][Hq][T][3]; all in dtype.  block_idx [B][Hkv][T][S] int32,
 * S = min(n_sel, T / sel_block): read when idx_given, else written (top-S
 * of the importance, ties to the lower block).  out [B][Hq][T][D] in dtype.
 * Requires T >= cmp_block and T >= sel_block.  Two caller buffers: ctx
 * (nsa_fused_ctx_bytes) is written by the forward and read by the backward
 * (pooled keys, packed q, the float32 branch outputs, their lse, the block ->
 * query CSR); scratch (nsa_fused_scratch_bytes, for the stream's device) is
 * transient and may be shared by both calls.  The backward takes the
 * forward's inputs again, dO, and writes every gradient in dtype: dq, dkc /
 * dvc (shaped like kc / vc), dks, dvs, dkw, dvw, dgate [B][Hq][T][3]; the
 * compression and selection dK/dV use the deterministic partial merge. */
size_t nsa_fused_ctx_bytes(int B, int Hq, int Hkv, int T, int D, int cmp_block, int cmp_stride, int sel_block,
                           int n_sel, int window, int pooled, int dtype);
size_t nsa_fused_scratch_bytes(int B, int Hq, int Hkv, int T, int D, int cmp_block, int cmp_stride, int sel_block,
                               int n_sel, int window, int pooled, int dtype, void* stream);
int nsa_fused_fwd(const void* q, const void* kc, const void* vc, const void* ks, const void* vs, const void* kw,
                  const void* vw, const void* gate, int32_t* block_idx, int idx_given, void* out, void* ctx,
                  size_t ctx_bytes, void* scratch, size_t scratch_bytes, int B, int Hq, int Hkv, int T, int D,
                  int cmp_block, int cmp_stride, int sel_block, int n_sel, int window, int force_init, int n_local,
                  int pooled, int dtype, void* stream);
int nsa_fused_bwd(const void* dout, const void* q, const void* kc, const void* vc, const void* ks, const void* vs,
                  const void* kw, const void* vw, const void* gate, const int32_t* block_idx, const void* ctx,
                  size_t ctx_bytes, void* scratch, size_t scratch_bytes, void* dq, void* dkc, void* dvc, void* dks,
                  void* dvs, void* dkw, void* dvw, void* dgate, int B, int Hq, int Hkv, int T, int D, int cmp_block,
                  int cmp_stride, int sel_block, int n_sel, int window, int pooled, int dtype, void* stream);

/* ---- block importance + top-n ----------------------------------------------
 * Replaces the importance / topk block of NSAAttention._forward_fused
 * (nsa_model.py:343-355): p_cmp = exp(q.k_cmp*scale - lse_cmp) summed over
 * each GQA group, mapped to selection blocks by span overlap / cmp_stride,
 * non-causal blocks set to -FLT_MAX, forced blocks (block 0 if force_init,
 * the n_local most recent blocks) set to +inf, then top-S with ties to the
 * lower block index.  S = min(n_sel, T / sel_block).  scores (nullable,
 * float [B][Hkv][T][T/sel_block]) receives the raw importance. */
int nsa_importance_topn(const void* q, const void* k_cmp, const float* lse_cmp, int32_t* block_idx,
                        float* scores, int B, int Hq, int Hkv, int T, int n_cmp, int D, int cmp_block,
                        int cmp_stride, int sel_block, int n_sel, int force_init, int n_local, int dtype,
                        void* stream);

/* ---- compression phi (NSA paper eq. 7) --------------------------------------
 * Replaces BlockCompressor (nsa_model.py:100-123), the reference's weighted
 * mean + linear, by the paper's learnable MLP over each span of l tokens at
 * stride d with an intra-block position encoding P:
 *   out[i] = W2 silu(W1 vec(x[i d .. i d + l - 1] + P) + b1) + b2
 * x [BH][L][D] (spans read in place), w1 [H][l D], w2 [D][H] in dtype;
 * c1 = b1 + W1 vec(P) and b2 float [H] / [D]; out [BH][n][D] in dtype with
 * n = (L - l)/d + 1; pre (float [BH][n][H]) receives W1 vec(span + P) + b1 for
 * the backward.  D in {64, 128}, H in {32, 64, 128}. */
int nsa_phi_fwd(const void* x, const void* w1, const float* c1, const void* w2, const float* b2, void* out,
                float* pre, int BH, int L, int D, int H, int l, int d, int dtype, void* stream);
/* Backward of phi's hidden layer: dpre = (W2^T dout) * silu'(pre).  dout
 * [BH][n][D] and w2t = W2^T [H][D] in dtype; pre / dpre float [BH][n][H]. */
int nsa_phi_dpre(const void* dout, const void* w2t, const float* pre, float* dpre, int BH, int n, int D, int H,
                 int dtype, void* stream);
/* Gradient of the spans back onto the sequence: dx[p] = sum over the spans i
 * holding p (i d <= p < i d + l) of dspan[i][(p - i d) D ..], spans ascending,
 * summed in float (deterministic).  dspan [BH][n][l D] in dspan_dtype; dx
 * [BH][L][D] in dx_dtype. */
int nsa_phi_fold(const void* dspan, int dspan_dtype, void* dx, int BH, int L, int D, int l, int d, int dx_dtype,
                 void* stream);
/* Parameter gradients of phi (the reference trains its pooler's weights by
 * autograd, nsa_model.py:100-123), over the n pooled tokens of every
 * sequence: dW1 = sum dpre^T vec(span + P) [H][l D], dW2 = sum dout^T
 * silu(pre) [D][H], db1 / db2 the column sums of dpre / dout, dpos = db1^T W1
 * as [l][D]; all float.  x [BH][L][D] and dout [BH][n][D] in dtype, dpre / pre
 * float [BH][n][H], pos float [l][D], w1 float [H][l D].  The spans are read
 * in place.  The tokens are summed in ranges fixed by the shape, then the
 * ranges in order: the same bits on every run.  workspace: at least
 * nsa_phi_wgrad_workspace(BH, n, D, H, l) bytes (0: unsupported shape).
 * D in {64, 128}, H in {32, 64, 128}. */
size_t nsa_phi_wgrad_workspace(int BH, int n, int D, int H, int l);
int nsa_phi_wgrad(const void* x, const void* dout, const float* dpre, const float* pre, const float* pos,
                  const float* w1, float* dw1, float* db1, float* dw2, float* db2, float* dpos, void* workspace,
                  size_t workspace_bytes, int BH, int L, int D, int H, int l, int d, int dtype, void* stream);

/* ---- decode: one new query per sequence against its KV caches ---------------
 * No reference counterpart as an entry point: the reference runs whole
 * sequences only (NSAAttention.forward, nsa_model.py:196-304).  A decode step
 * computes that function's row t = lens[b] - 1 for every sequence b, with the
 * candidate blocks 0 .. t / sel_block (the row of a prefill whose length
 * reaches the end of t's selection block):
 *   q, out            [B][Hq][D]
 *   k_cmp, v_cmp      [B][Hkv][Ncap][D]  pooled caches (nsa_pool_fwd of kc / vc)
 *   ks vs kw vw       [B][Hkv][Tcap][D]  branch caches; rows >= lens[b] unread
 *   gate              [B][Hq][3] logits
 *   lens              [B] int32 on the device, 0 <= lens[b] <= Tcap
 *   block_idx (out)   [B][Hkv][n_sel] int32, -1 past S = min(n_sel, t/sel_block + 1)
 *   scores (nullable) float [B][Hkv][(Tcap-1)/sel_block + 1]: raw importance
 *                     of blocks 0 .. t/sel_block
 *   o_branch (nullable) float [3][B][Hq][D]: compression, selection, window
 *   lse_branch (nullable) float [3][B][Hq]
 * Ncap >= (Tcap - cmp_block)/cmp_stride + 1 and (Tcap-1)/sel_block + 1 <= 4096.
 * workspace: 256-byte aligned, at least nsa_decode_workspace() bytes (0 =
 * unsupported shape); it carries the split partials between the launches. */
size_t nsa_decode_workspace(int B, int Hq, int Hkv, int D, int Tcap, int Ncap, int cmp_block, int cmp_stride,
                            int sel_block, int n_sel, int window);
int nsa_decode_fwd(const void* q, const void* k_cmp, const void* v_cmp, const void* ks, const void* vs,
                   const void* kw, const void* vw, const void* gate, const int32_t* lens, void* out,
                   int32_t* block_idx, float* scores, float* o_branch, float* lse_branch, void* workspace,
                   size_t workspace_bytes, int B, int Hq, int Hkv, int D, int Tcap, int Ncap, int cmp_block,
                   int cmp_stride, int sel_block, int n_sel, int window, int force_init, int n_local, int dtype,
                   void* stream);

/* Append one token per sequence to the decode caches (no reference
 * counterpart; the cache update a decode loop needs between steps): the six
 * new rows [B][Hkv][D] go to position lens_in[b] of kc vc ks vs kw vw, and
 * when the new length completes a pooled span the pooled token of kc / vc is
 * written to k_cmp / v_cmp exactly as nsa_pool_fwd computes it.
 * lens_out[b] = lens_in[b] + 1 (unchanged, and nothing written, when the
 * cache is full).  lens_in and lens_out must be different buffers. */
int nsa_decode_append(void* kc, void* vc, void* ks, void* vs, void* kw, void* vw, void* k_cmp, void* v_cmp,
                      const void* kc_new, const void* vc_new, const void* ks_new, const void* vs_new,
                      const void* kw_new, const void* vw_new, const int32_t* lens_in, int32_t* lens_out, int B,
                      int Hkv, int D, int Tcap, int Ncap, int cmp_block, int cmp_stride, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSA_HIP_H */
