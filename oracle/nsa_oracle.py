"""CPU restatement of the reference NSA attention semantics.

TEST INFRASTRUCTURE ONLY.  This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and never as the thing that is measured or shipped.  The product
path (``openbox-llm_amd/``) never imports it and fails loudly when its HIP
library is missing.

Everything here is plain PyTorch on the CPU, float64 by default (float32 for
the timed CPU baseline).  Each function cites the reference file:line whose
behaviour it restates (paths relative to the reference checkout).

Semantic contract (shared with the HIP kernels)
-----------------------------------------------
Layout ``q [B,Hq,T,D]``, ``k/v [B,Hkv,T,D]``; query head ``h`` reads KV head
``h // G`` with ``G = Hq // Hkv`` (nsa_model.py:85-93).  ``scale = D**-0.5``
(nsa_model.py:164, nsa_selection_kernel.py:210).

* compression: pooled token ``i`` is the mean of ``k[i*d : i*d+l]``
  (nsa_fused_kernel.py:549-554 is the aligned case ``l = d``); token ``i`` is
  visible to query ``t`` iff ``i*d + l - 1 <= t`` (nsa_model.py:233-235,
  nsa_fused_kernel.py:88).
* window: keys ``t-w < p <= t`` (nsa_model.py:287-289).
* selection: keys of the selected blocks ``[j*ls, (j+1)*ls)`` with ``p <= t``
  and ``p < T`` (nsa_selection_kernel.py:141-146).  Rows with no visible key
  produce 0 and ``lse = -1e9`` (nsa_model.py:70-82,
  nsa_selection_kernel.py:165-172).
* importance: ``imp_cmp[t,i] = sum_g p_cmp[hkv*G+g, t, i]`` (nsa_model.py:250)
  mapped onto selection blocks by overlap weight ``|span_i & block_j| / d``
  (identity when ``l = d = ls``); non-causal blocks get ``finfo(f32).min``
  (nsa_model.py:253-254); forced blocks (block 0 and the two local blocks)
  get ``+inf``; top-S with S = min(n, n_slc) (nsa_model.py:257-258), ties to
  the lower block index (build-defined: ``torch.topk`` leaves tie order
  unspecified).
* gate: ``out = sum_c sigmoid(gate[...,c]) * o_c`` (nsa_model.py:293-301,
  nsa_fused_kernel.py:572-573).
* compression phi (``phi_compress``): the paper's MLP over each span with
  an intra-block position encoding (a widening of the reference's pooler).
* decode (``decode_reference``): row ``t = len-1`` of the above from caches,
  candidate blocks ``0 .. t // ls``; pinned against the whole-sequence
  functions in tests/test_oracle_pins.py.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

LSE_EMPTY = -1.0e9          # finite lse sentinel for rows with no visible key
F32_MIN = float(torch.finfo(torch.float32).min)


# ---------------------------------------------------------------------------
# configuration
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class NSAConfig:
    """Block geometry of the three branches.

    ``cmp_block``/``cmp_stride`` are the compression span ``l`` and stride
    ``d``; ``sel_block`` is the selection block ``l'``; ``n_sel`` the top-n
    count; ``window`` the sliding window ``w``.  ``force_init`` and
    ``n_local`` force block 0 and the ``n_local`` most recent blocks into the
    selection.  ``NSAConfig.reference(bs, n, w)`` is the reference's aligned
    grid (nsa_model.py:134-140): ``l = d = l' = bs`` and no forcing.
    """

    cmp_block: int
    cmp_stride: int
    sel_block: int
    n_sel: int
    window: int
    force_init: bool = False
    n_local: int = 0

    @staticmethod
    def reference(block_size: int, n_sel: int, window: int) -> "NSAConfig":
        return NSAConfig(block_size, block_size, block_size, n_sel, window)


def n_cmp_tokens(T: int, l: int, d: int) -> int:
    """Number of pooled tokens ``floor((T-l)/d)+1`` (``T//l`` when l == d,
    nsa_fused_kernel.py:551)."""
    return (T - l) // d + 1 if T >= l else 0


def n_sel_blocks(T: int, ls: int) -> int:
    """Complete selection blocks, ``T // ls`` (nsa_model.py:201)."""
    return T // ls


# ---------------------------------------------------------------------------
# compression pooling
# ---------------------------------------------------------------------------

def pool_mean(x: torch.Tensor, l: int, d: int) -> torch.Tensor:
    """Mean pool over spans ``[i*d, i*d+l)``: ``[B,H,T,D] -> [B,H,n,D]``.

    With ``l == d`` this is nsa_fused_kernel.py:549-554 (reshape + mean).
    """
    B, H, T, D = x.shape
    n = n_cmp_tokens(T, l, d)
    if n == 0:
        return x.new_zeros(B, H, 0, D)
    idx = (torch.arange(n)[:, None] * d + torch.arange(l)[None, :]).reshape(-1)
    return x[:, :, idx].reshape(B, H, n, l, D).mean(dim=3)


# ---------------------------------------------------------------------------
# masks
# ---------------------------------------------------------------------------

def phi_compress(x, pos, w1, b1, w2, b2, l: int, d: int, act: str = "silu") -> torch.Tensor:
    """The NSA paper's compression phi (arXiv:2502.11089, eq. 7), the
    alternative to the reference's weighted mean + linear
    (nsa_model.py:100-123): pooled token i of ``x [B,H,T,D]`` is
    ``w2 act(w1 vec(x[i*d : i*d+l] + pos) + b1) + b2`` (``vec`` flattens the
    span row-major, position-major), ``act`` SiLU or the identity."""
    B, H, T, D = x.shape
    n = n_cmp_tokens(T, l, d)
    spans = x[:, :, :(n - 1) * d + l].unfold(2, l, d).transpose(-1, -2) if n > 0 else x.new_zeros(B, H, 0, l, D)
    z = (spans + pos).reshape(B, H, n, l * D)
    a = z @ w1.transpose(0, 1) + b1
    hdn = a * torch.sigmoid(a) if act == "silu" else a
    return hdn @ w2.transpose(0, 1) + b2


def window_keep(T: int, w: int) -> torch.Tensor:
    """``[T,T]`` band mask ``p <= t and t - p < w`` (nsa_model.py:287-289)."""
    t = torch.arange(T)[:, None]
    p = torch.arange(T)[None, :]
    return (p <= t) & (t - p < w)


def compress_keep(T: int, n: int, l: int, d: int) -> torch.Tensor:
    """``[T,n]``: pooled token ``i`` visible iff ``i*d + l - 1 <= t``
    (nsa_model.py:233-235 with l = d)."""
    t = torch.arange(T)[:, None]
    i = torch.arange(n)[None, :]
    return i * d + l - 1 <= t


def select_keep(block_idx: torch.Tensor, T: int, ls: int) -> torch.Tensor:
    """``[B,Hkv,T,T]`` token mask of the selected blocks, causal
    (nsa_selection_kernel.py:74-85; tokens past the block grid are only
    reached through their own block, matching the kernel at :141-146)."""
    B, Hkv, Tq, S = block_idx.shape
    p = torch.arange(T)
    blk_of_p = p // ls                                          # [T]
    idx = block_idx.long()
    chosen = (idx[..., :, None] == blk_of_p[None, None, None, None, :]) \
        & (idx[..., :, None] >= 0)                              # [B,Hkv,T,S,T]
    keep = chosen.any(dim=3)
    causal = p[None, :] <= torch.arange(Tq)[:, None]
    return keep & causal[None, None]


# ---------------------------------------------------------------------------
# dense masked attention (small T)
# ---------------------------------------------------------------------------

def expand_kv(x: torch.Tensor, G: int) -> torch.Tensor:
    """GQA expansion, head h -> KV head h // G (nsa_model.py:85-93)."""
    return x.repeat_interleave(G, dim=1)


def masked_attention(q, k, v, keep, scale=None):
    """Softmax attention restricted to ``keep``; empty rows give 0.

    ``q [B,Hq,T,D]``, ``k/v [B,Hkv,Lk,D]``, ``keep`` broadcastable to
    ``[B,Hkv,T,Lk]``.  Returns ``(o, lse)``, ``lse [B,Hq,T]`` natural-log
    sum-exp of the scaled scores with ``LSE_EMPTY`` on empty rows.  This is
    masked_softmax (nsa_model.py:70-82) followed by ``p @ v``; the finite
    fill of the reference never wins over a visible key, so masking with -inf
    here is the same function.
    """
    B, Hq, T, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    keep = torch.as_tensor(keep).expand(B, Hkv, T, Lk)
    keep_h = expand_kv(keep, G)
    s = torch.matmul(q, expand_kv(k, G).transpose(-1, -2)) * scale
    s = s.masked_fill(~keep_h, float("-inf"))
    has = keep_h.any(dim=-1)
    lse = torch.logsumexp(s, dim=-1)
    lse = torch.where(has, lse, torch.full_like(lse, LSE_EMPTY))
    p = torch.exp(s - lse[..., None]).masked_fill(~keep_h, 0.0)
    o = torch.matmul(p, expand_kv(v, G))
    return o, lse


def attention_probs(q, k, keep, scale=None):
    """Masked softmax probabilities ``[B,Hq,T,Lk]`` (nsa_model.py:70-82)."""
    B, Hq, T, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    keep_h = expand_kv(torch.as_tensor(keep).expand(B, Hkv, T, Lk), G)
    s = torch.matmul(q, expand_kv(k, G).transpose(-1, -2)) * scale
    s = s.masked_fill(~keep_h, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.nan_to_num(p, nan=0.0) * keep_h.any(dim=-1, keepdim=True)


def window_attention(q, k, v, w):
    T = q.shape[2]
    return masked_attention(q, k, v, window_keep(T, w)[None, None])


def compression_attention(q, k_cmp, v_cmp, l, d):
    T, n = q.shape[2], k_cmp.shape[2]
    return masked_attention(q, k_cmp, v_cmp, compress_keep(T, n, l, d)[None, None])


def selection_attention(q, k, v, block_idx, ls):
    T = q.shape[2]
    return masked_attention(q, k, v, select_keep(block_idx, T, ls))


# ---------------------------------------------------------------------------
# importance and top-n
# ---------------------------------------------------------------------------

def overlap_weights(n_cmp: int, n_slc: int, l: int, d: int, ls: int) -> torch.Tensor:
    """``W[i,j] = |[i*d, i*d+l) & [j*ls, (j+1)*ls)| / d`` as float64.

    For ``l = d = ls`` this is the identity, so importance(block j) is the
    compression probability of token j (nsa_model.py:245-250).  At
    l=32, d=16, ls=64 each block collects tokens 4j-1..4j+3 with weights
    1,2,2,2,1 (NSA paper, arXiv:2502.11089 eq. 9, cited at nsa_model.py:5-6).
    """
    i = torch.arange(n_cmp, dtype=torch.float64)[:, None]
    j = torch.arange(n_slc, dtype=torch.float64)[None, :]
    lo = torch.maximum(i * d, j * ls)
    hi = torch.minimum(i * d + l, (j + 1) * ls)
    return (hi - lo).clamp(min=0) / d


def importance(q, k_cmp, cfg: NSAConfig, T: int | None = None):
    """Raw block importance ``[B,Hkv,T,n_slc]`` (before masking/forcing).

    p_cmp of the compression branch summed over each GQA group
    (nsa_model.py:245-250) and mapped onto selection blocks by
    ``overlap_weights``.
    """
    B, Hq, Tq, D = q.shape
    Hkv = k_cmp.shape[1]
    G = Hq // Hkv
    T = Tq if T is None else T
    n = k_cmp.shape[2]
    n_slc = n_sel_blocks(T, cfg.sel_block)
    if n == 0 or n_slc == 0:
        return q.new_zeros(B, Hkv, Tq, n_slc)
    keep = compress_keep(Tq, n, cfg.cmp_block, cfg.cmp_stride)[None, None]
    p = attention_probs(q, k_cmp, keep)                         # [B,Hq,T,n]
    imp_cmp = p.reshape(B, Hkv, G, Tq, n).sum(dim=2)            # [B,Hkv,T,n]
    W = overlap_weights(n, n_slc, cfg.cmp_block, cfg.cmp_stride,
                        cfg.sel_block).to(imp_cmp.dtype)
    return imp_cmp @ W


def selection_scores(imp, cfg: NSAConfig, t_pos=None):
    """Mask and force the raw importance: the top-n input.

    Non-causal blocks (``(j+1)*ls - 1 > t``) get ``finfo(f32).min``
    (nsa_model.py:253-254); forced blocks (block 0 if ``force_init``; blocks
    ``t//ls - m`` for ``m < n_local``) get ``+inf``.  ``t_pos`` gives the query
    position of each row (default ``arange(T)``).
    """
    B, Hkv, R, n_slc = imp.shape
    ls = cfg.sel_block
    t = torch.arange(R) if t_pos is None else torch.as_tensor(t_pos)
    j = torch.arange(n_slc)
    valid = (j[None, :] + 1) * ls - 1 <= t[:, None]             # [R,n_slc]
    sc = imp.to(torch.float64).masked_fill(~valid[None, None], F32_MIN)
    forced = torch.zeros(R, n_slc, dtype=torch.bool)
    if cfg.force_init and n_slc > 0:
        forced[:, 0] = True
    for m in range(cfg.n_local):
        jl = t // ls - m
        ok = (jl >= 0) & (jl < n_slc)
        forced[torch.arange(R)[ok], jl[ok]] = True
    return sc.masked_fill(forced[None, None], float("inf"))


def topn_from_scores(scores, S: int) -> torch.Tensor:
    """Top-S block indices per row: descending score, ties to the lower index.

    Replaces ``torch.topk(imp, S).indices`` (nsa_model.py:258, :355); a stable
    descending sort fixes the tie order that topk leaves open.
    """
    order = torch.sort(scores, dim=-1, descending=True, stable=True).indices
    return order[..., :S].to(torch.int32)


def select_blocks(q, k_cmp, cfg: NSAConfig):
    """Importance -> mask/force -> top-n: ``(block_idx, raw_importance)``."""
    T = q.shape[2]
    n_slc = n_sel_blocks(T, cfg.sel_block)
    S = min(cfg.n_sel, n_slc)
    imp = importance(q, k_cmp, cfg)
    return topn_from_scores(selection_scores(imp, cfg), S), imp


# ---------------------------------------------------------------------------
# gate and the three-branch forward
# ---------------------------------------------------------------------------

def gate_blend(gate_logits, o_cmp, o_slc, o_win):
    """``sum_c sigmoid(g_c) * o_c`` (nsa_model.py:293-301)."""
    g = torch.sigmoid(gate_logits)
    return g[..., 0:1] * o_cmp + g[..., 1:2] * o_slc + g[..., 2:3] * o_win


def nsa_fused_reference(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx,
                        cfg: NSAConfig):
    """Three-branch gated NSA with given block indices.

    nsa_fused_kernel.py:600-609 generalised to the l/d/ls geometry.  Returns
    ``(out, parts)`` where ``parts`` holds each branch's ``(o, lse)``.
    """
    T = q.shape[2]
    k_cmp = pool_mean(kc, cfg.cmp_block, cfg.cmp_stride)
    v_cmp = pool_mean(vc, cfg.cmp_block, cfg.cmp_stride)
    o_c, lse_c = compression_attention(q, k_cmp, v_cmp, cfg.cmp_block, cfg.cmp_stride)
    if block_idx.shape[-1] > 0:
        o_s, lse_s = selection_attention(q, ks, vs, block_idx, cfg.sel_block)
    else:
        o_s = torch.zeros_like(q)
        lse_s = torch.full(q.shape[:3], LSE_EMPTY, dtype=q.dtype)
    o_w, lse_w = window_attention(q, kw, vw, cfg.window)
    out = gate_blend(gate_logits, o_c, o_s, o_w)
    return out, {"cmp": (o_c, lse_c), "slc": (o_s, lse_s), "win": (o_w, lse_w),
                 "k_cmp": k_cmp, "v_cmp": v_cmp}


def nsa_forward_reference(q, kc, vc, ks, vs, kw, vw, gate_logits, cfg: NSAConfig):
    """Full NSA: block indices from the compression importance, then the
    three gated branches (nsa_model.py:196-304 at the attention level)."""
    k_cmp = pool_mean(kc, cfg.cmp_block, cfg.cmp_stride)
    with torch.no_grad():
        block_idx, imp = select_blocks(q.detach(), k_cmp.detach(), cfg)
    out, parts = nsa_fused_reference(q, kc, vc, ks, vs, kw, vw, gate_logits,
                                     block_idx, cfg)
    parts["block_idx"] = block_idx
    parts["importance"] = imp
    return out, parts


# ---------------------------------------------------------------------------
# analytic backward (restating nsa_selection_backward.py:12-20)
# ---------------------------------------------------------------------------

def attention_backward(q, k, v, keep, do, scale=None):
    """Closed-form gradients of ``masked_attention``.

    ``delta_i = sum_d dO_i O_i``; ``dS = P * (dO V^T - delta)``;
    ``dQ = scale dS K``; ``dK = scale dS^T Q``; ``dV = P^T dO``
    (nsa_selection_backward.py:12-20, delta at :168).  GQA heads of a group
    accumulate into their shared KV head.
    """
    B, Hq, T, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    p = attention_probs(q, k, keep, scale)                      # [B,Hq,T,Lk]
    ke, ve = expand_kv(k, G), expand_kv(v, G)
    o = p @ ve
    delta = (do * o).sum(-1, keepdim=True)
    ds = p * (do @ ve.transpose(-1, -2) - delta)
    dq = scale * ds @ ke
    dk = (scale * ds.transpose(-1, -2) @ q).reshape(B, Hkv, G, Lk, D).sum(2)
    dv = (p.transpose(-1, -2) @ do).reshape(B, Hkv, G, Lk, D).sum(2)
    return dq, dk, dv


# ---------------------------------------------------------------------------
# block -> query CSR (restating nsa_fsa.py:14-64)
# ---------------------------------------------------------------------------

def build_block_to_query_csr(block_idx, block_size, n_blk=None):
    """Invert ``block_idx [B,Hkv,T,S]`` into a causal block -> query CSR.

    Every slot (t, s) with ``j = block_idx[..., t, s] >= 0`` and
    ``j*block_size <= t`` is one pair (nsa_fsa.py:40-42; a block listed twice
    in a row gives two pairs).  Pairs are grouped by (b, hkv, j) in slot order,
    i.e. queries ascending (stable order, nsa_fsa.py:58-62), with global
    offsets.  Returns int32 ``(q_of_block [P], block_offsets [B,Hkv,n_blk+1],
    pair_bh [P])``.

    ``n_blk`` defaults to the reference's ``T // block_size`` (nsa_fsa.py:36);
    a causal pair on a block at or past it raises IndexError, as the
    reference's ``scatter_add_`` into ``n_blk`` columns does (nsa_fsa.py:46-48).
    ``n_blk = ceil(T / block_size)`` covers the trailing partial block.
    """
    B, Hkv, T, S = block_idx.shape
    if n_blk is None:
        n_blk = T // block_size
    idx = block_idx.long()
    tpos = torch.arange(T)[None, None, :, None]
    valid = (idx >= 0) & (idx * block_size <= tpos)
    if bool((valid & (idx >= n_blk)).any()):
        raise IndexError(f"block index >= n_blk = {n_blk} on a causal pair")
    bh = (torch.arange(B)[:, None] * Hkv + torch.arange(Hkv)[None, :])[:, :, None, None]
    keys = (bh * n_blk + idx).expand(B, Hkv, T, S)[valid]        # (b, hkv, t, s) order
    vals = tpos.expand(B, Hkv, T, S)[valid]
    order = torch.sort(keys, stable=True).indices
    q_of_block = vals[order]
    pair_bh = keys[order] // max(n_blk, 1)
    counts = torch.bincount(keys, minlength=B * Hkv * n_blk) if keys.numel() else \
        torch.zeros(B * Hkv * n_blk, dtype=torch.int64)
    starts = torch.zeros(B * Hkv * n_blk + 1, dtype=torch.int64)
    starts[1:] = counts.cumsum(0)
    rows = torch.arange(B * Hkv)[:, None] * n_blk + torch.arange(n_blk + 1)[None, :]
    offsets = starts[rows].reshape(B, Hkv, n_blk + 1)
    return q_of_block.to(torch.int32), offsets.to(torch.int32), pair_bh.to(torch.int32)


# ---------------------------------------------------------------------------
# row-sampled evaluation (large T: parity on sampled rows, CPU baseline)
# ---------------------------------------------------------------------------

def _row_softmax_attention(s, m, vg_fn):
    """Softmax over the last axis of scaled scores ``s`` restricted to ``m``;
    ``vg_fn(p)`` contracts the probabilities with the values.  Empty rows
    give 0 and ``LSE_EMPTY`` (nsa_model.py:70-82)."""
    s = s.masked_fill(~m, float("-inf"))
    has = m.any(-1)
    lse = torch.logsumexp(s, dim=-1)
    lse = torch.where(has, lse, torch.full_like(lse, LSE_EMPTY))
    p = torch.exp(s - lse[..., None]).masked_fill(~m, 0.0)
    return vg_fn(p), lse


def _gathered_attention(q_rows, k, v, kidx, kmask, scale):
    """Attention of ``q_rows [B,Hq,R,D]`` over gathered keys ``kidx [B,Hkv,R,K]``."""
    B, Hq, R, D = q_rows.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    safe = kidx.clamp(min=0, max=k.shape[2] - 1)   # masked slots may point past the keys
    bi = torch.arange(B)[:, None, None, None]
    hi = torch.arange(Hkv)[None, :, None, None]
    kg = k[bi, hi, safe]                                        # [B,Hkv,R,K,D]
    vg = v[bi, hi, safe]
    qg = q_rows.reshape(B, Hkv, G, R, D)
    s = torch.einsum("bhgrd,bhrkd->bhgrk", qg, kg) * scale
    o, lse = _row_softmax_attention(s, kmask[:, :, None],
                                    lambda p: torch.einsum("bhgrk,bhrkd->bhgrd", p, vg))
    return o.reshape(B, Hq, R, D), lse.reshape(B, Hq, R)


def _shared_key_attention(q_rows, k, v, kmask, scale):
    """Attention of ``q_rows [B,Hq,R,D]`` over all of ``k/v [B,Hkv,n,D]``
    restricted to ``kmask [R,n]`` (the pooled keys are shared by every row,
    so no gather is needed)."""
    B, Hq, R, D = q_rows.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    qg = q_rows.reshape(B, Hkv, G * R, D)
    s = (qg @ k.transpose(-1, -2)).reshape(B, Hkv, G, R, -1) * scale
    o, lse = _row_softmax_attention(
        s, kmask[None, None, None],
        lambda p: (p.reshape(B, Hkv, G * R, -1) @ v).reshape(B, Hkv, G, R, D))
    return o.reshape(B, Hq, R, D), lse.reshape(B, Hq, R)


def nsa_rows(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, cfg: NSAConfig,
             rows, k_cmp=None, v_cmp=None):
    """Three-branch output for the query positions ``rows`` only.

    Same function as ``nsa_fused_reference`` restricted to those rows, with
    the keys of each row gathered explicitly (window range, selected blocks;
    the visible pooled tokens by mask).  Memory is O(rows * keys) instead of
    O(T^2), so it serves T = 32K parity sampling and the CPU baseline.
    """
    rows = torch.as_tensor(rows, dtype=torch.long)
    return nsa_rows_gathered(q[:, :, rows], kc, vc, ks, vs, kw, vw, gate_logits[:, :, rows],
                             block_idx[:, :, rows], cfg, rows, q.shape[2], k_cmp, v_cmp)


def nsa_rows_gathered(q_rows, kc, vc, ks, vs, kw, vw, gate_rows, idx_rows, cfg: NSAConfig,
                      rows, T, k_cmp=None, v_cmp=None):
    """``nsa_rows`` with the row inputs already gathered: ``q_rows
    [B,Hq,R,D]``, ``gate_rows [B,Hq,R,3]`` and ``idx_rows [B,Hkv,R,S]`` are
    the values at the query positions ``rows`` of a length-``T`` sequence
    (so gradients of ``q_rows`` / ``gate_rows`` are per-row tensors)."""
    B, Hq, R, D = q_rows.shape
    scale = D ** -0.5
    rows = torch.as_tensor(rows, dtype=torch.long)
    assert rows.numel() == R
    Hkv = kc.shape[1]
    if k_cmp is None:
        k_cmp = pool_mean(kc, cfg.cmp_block, cfg.cmp_stride)
    if v_cmp is None:
        v_cmp = pool_mean(vc, cfg.cmp_block, cfg.cmp_stride)
    qr = q_rows
    # window
    w = cfg.window
    off = torch.arange(w)
    kidx = rows[:, None] - (w - 1) + off[None, :]               # [R,w]
    km = kidx >= 0
    o_w, lse_w = _gathered_attention(qr, kw, vw, kidx.expand(B, Hkv, R, w),
                                     km.expand(B, Hkv, R, w), scale)
    # compression
    n = k_cmp.shape[2]
    if n > 0:
        ci = torch.arange(n)
        cm = (ci[None, :] * cfg.cmp_stride + cfg.cmp_block - 1) <= rows[:, None]
        o_c, lse_c = _shared_key_attention(qr, k_cmp, v_cmp, cm, scale)
    else:
        o_c = torch.zeros_like(qr)
        lse_c = torch.full((B, Hq, R), LSE_EMPTY, dtype=qr.dtype)
    # selection
    S = idx_rows.shape[-1]
    ls = cfg.sel_block
    if S > 0:
        bl = idx_rows.long()                                    # [B,Hkv,R,S]
        pos = bl[..., None] * ls + torch.arange(ls)             # [B,Hkv,R,S,ls]
        pm = (bl[..., None] >= 0) & (pos <= rows[None, None, :, None, None]) & (pos < T)
        o_s, lse_s = _gathered_attention(qr, ks, vs, pos.reshape(B, Hkv, R, S * ls),
                                         pm.reshape(B, Hkv, R, S * ls), scale)
    else:
        o_s = torch.zeros_like(qr)
        lse_s = torch.full((B, Hq, R), LSE_EMPTY, dtype=qr.dtype)
    out = gate_blend(gate_rows, o_c, o_s, o_w)
    return out, {"cmp": (o_c, lse_c), "slc": (o_s, lse_s), "win": (o_w, lse_w)}


def selection_rows(q_rows, k, v, idx_rows, ls, rows, T):
    """Selection-branch ``(o, lse)`` of the query positions ``rows`` only
    (the selection part of ``nsa_rows_gathered``; nsa_selection_kernel.py:55-92
    restricted to those rows)."""
    B, Hq, R, D = q_rows.shape
    Hkv = k.shape[1]
    rows = torch.as_tensor(rows, dtype=torch.long)
    S = idx_rows.shape[-1]
    bl = idx_rows.long()
    pos = bl[..., None] * ls + torch.arange(ls)
    pm = (bl[..., None] >= 0) & (pos <= rows[None, None, :, None, None]) & (pos < T)
    return _gathered_attention(q_rows, k, v, pos.reshape(B, Hkv, R, S * ls), pm.reshape(B, Hkv, R, S * ls),
                               D ** -0.5)


def importance_rows(q, k_cmp, cfg: NSAConfig, rows, T):
    """Raw importance ``[B,Hkv,R,n_slc]`` for the query positions ``rows``."""
    rows = torch.as_tensor(rows, dtype=torch.long)
    return importance_gathered(q[:, :, rows], k_cmp, cfg, rows, T)


def importance_gathered(q_rows, k_cmp, cfg: NSAConfig, rows, T):
    """``importance_rows`` with the query rows already gathered: ``q_rows
    [B,Hq,R,D]`` are the queries at positions ``rows`` of a length-``T``
    sequence (nsa_model.py:245-250 restricted to those rows)."""
    B, Hq, R, D = q_rows.shape
    Hkv = k_cmp.shape[1]
    G = Hq // Hkv
    rows = torch.as_tensor(rows, dtype=torch.long)
    n = k_cmp.shape[2]
    n_slc = n_sel_blocks(T, cfg.sel_block)
    keep = (torch.arange(n)[None, :] * cfg.cmp_stride + cfg.cmp_block - 1) <= rows[:, None]
    p = attention_probs(q_rows, k_cmp, keep[None, None])
    imp_cmp = p.reshape(B, Hkv, G, R, n).sum(2)
    W = overlap_weights(n, n_slc, cfg.cmp_block, cfg.cmp_stride, cfg.sel_block)
    return imp_cmp @ W.to(imp_cmp.dtype)


# ---------------------------------------------------------------------------
# decode: one new query per sequence against its caches
# ---------------------------------------------------------------------------

def decode_reference(q, kc, vc, ks, vs, kw, vw, gate, lens, cfg: NSAConfig):
    """One decode step: row ``t = lens[b] - 1`` of the three-branch NSA for
    every sequence ``b`` (nsa_model.py:196-304 at that row).

    ``q [B,Hq,D]`` and ``gate [B,Hq,3]`` are the new query's; the caches
    ``kc..vw [B,Hkv,Tcap,D]`` are read below ``lens[b]`` only.  The candidate
    blocks are ``0 .. t // ls`` -- the row of a prefill whose length reaches
    the end of t's selection block, so a decode step does not depend on how
    long the sequence will grow.  Returns ``(out [B,Hq,D], block_idx
    [B,Hkv,n_sel] (-1 past S), parts)``; ``parts`` holds per sequence the raw
    importance of the candidates and each branch's ``(o, lse)``.
    """
    B, Hq, D = q.shape
    Hkv = kc.shape[1]
    ls = cfg.sel_block
    out = torch.zeros_like(q)
    idx = torch.full((B, Hkv, cfg.n_sel), -1, dtype=torch.int32)
    parts = []
    for b in range(B):
        n = int(lens[b])
        t = n - 1
        if t < 0:
            parts.append(None)
            continue
        ncand = t // ls + 1
        S = min(cfg.n_sel, ncand)
        sl = slice(b, b + 1)
        kcb, vcb = kc[sl, :, :n], vc[sl, :, :n]
        k_cmp = pool_mean(kcb, cfg.cmp_block, cfg.cmp_stride)
        v_cmp = pool_mean(vcb, cfg.cmp_block, cfg.cmp_stride)
        qb = q[sl, :, None, :]
        imp = importance_gathered(qb, k_cmp, cfg, [t], ncand * ls)     # [1,Hkv,1,ncand]
        pick = topn_from_scores(selection_scores(imp, cfg, t_pos=[t]), S)
        idx[b, :, :S] = pick[0, :, 0]
        o, br = nsa_rows_gathered(qb, kcb, vcb, ks[sl, :, :n], vs[sl, :, :n], kw[sl, :, :n], vw[sl, :, :n],
                                  gate[sl, :, None, :], pick, cfg, [t], n, k_cmp, v_cmp)
        out[b] = o[0, :, 0]
        parts.append({"importance": imp[0, :, 0], **{k: (v[0][0, :, 0], v[1][0, :, 0]) for k, v in br.items()}})
    return out, idx, parts


# ---------------------------------------------------------------------------
# algorithmic work (FLOP accounting shared with the bench)
# ---------------------------------------------------------------------------

def keys_per_row(T: int, cfg: NSAConfig, block_idx=None):
    """Visible keys per query for each branch.

    ``K_win(t) = min(w, t+1)``; ``K_cmp(t) = #{i : i*d+l-1 <= t}``;
    ``K_sel(b,hkv,t)`` counts the visible tokens of the actual selected
    blocks (or the nominal ``min(n*ls, t+1)`` without indices).
    Returns int64 totals ``(sum_win, sum_cmp, sum_sel)`` over one KV head's
    rows (selection summed over all ``(b, hkv)`` rows when indices are given).
    """
    t = torch.arange(T, dtype=torch.int64)
    k_win = torch.clamp(t + 1, max=cfg.window)
    n = n_cmp_tokens(T, cfg.cmp_block, cfg.cmp_stride)
    k_cmp = torch.clamp((t - cfg.cmp_block + 1) // cfg.cmp_stride + 1, min=0, max=n)
    k_cmp = torch.where(t >= cfg.cmp_block - 1, k_cmp, torch.zeros_like(k_cmp))
    if block_idx is None:
        k_sel = torch.clamp(t + 1, max=cfg.n_sel * cfg.sel_block).sum()
    else:
        bl = block_idx.long()
        ls = cfg.sel_block
        start = bl * ls
        vis = torch.clamp(torch.minimum(t[None, None, :, None] + 1, start + ls) - start,
                          min=0)
        vis = torch.where(bl >= 0, torch.clamp(torch.minimum(vis, T - start), min=0),
                          torch.zeros_like(vis))
        k_sel = vis.sum()
    return int(k_win.sum()), int(k_cmp.sum()), int(k_sel)
