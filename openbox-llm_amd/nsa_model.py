"""One NSA attention layer with the reference's ``attn_impl`` switch
(drop-in for ``NSAAttention`` of the reference module nsa_model.py:130-370).

* ``attn_impl='ref'``: the dense torch definition of the layer (nsa_model.py:196-304):
  three masked ``[B,Hq,T,T]`` attentions over the same projections.  It runs
  on any device and is the definition the fused path is checked against.
* ``attn_impl='fused'``: the same layer with the attention on the MI355X HIP
  kernels: compression attention over the learned pooled tokens, block
  importance + top-n, selection, sliding window and the gate blend in one
  autograd boundary (``nsa_hip_ops.NSAFusedHIP``).  The library is loaded on
  first use and its absence raises; nothing falls back to the 'ref' path.

Parameters, their names and their initialisation follow the reference
(nsa_model.py:147-195), so a reference ``state_dict`` loads unchanged.  The
block grid is the reference's aligned one: compression and selection share
``block_size``, pooled token j summarises block j.  Block choice in both paths
ranks blocks by descending importance and, among equal scores, by ascending
block index.  The reference's ``torch.topk`` leaves that order open; it only
matters on rows with fewer complete blocks than ``n_selected_blocks``, where
the masked fillers tie.  ``forward(x, block_idx=...)`` takes an explicit block
choice ``[B,Hkv,T,S]`` (-1 = empty slot) instead, e.g. one recorded from the
reference.
"""

import torch
import torch.nn as nn

__all__ = ["masked_softmax", "expand_kv", "BlockCompressor", "NSAAttention"]


def masked_softmax(scores, keep_mask):
    """Softmax over the last dim restricted to ``keep_mask``; rows with no kept
    position come out as zeros (nsa_model.py:70-82)."""
    filled = scores.masked_fill(~keep_mask, torch.finfo(scores.dtype).min)
    return torch.softmax(filled, dim=-1) * keep_mask.any(dim=-1, keepdim=True)


def expand_kv(x, group_size):
    """``[B,Hkv,S,D] -> [B,Hkv*G,S,D]``; query head h reads KV head h // G
    (nsa_model.py:85-93)."""
    return x.repeat_interleave(group_size, dim=1)


class BlockCompressor(nn.Module):
    """Learned pooling of one block of ``block_size`` tokens into one token:
    ``proj(sum_p softmax(pool_logits)_p * (x_p + intra_pos_p))``
    (nsa_model.py:100-123).  ``pool_logits`` start at zero, i.e. a plain mean."""

    def __init__(self, block_size, d_head):
        super().__init__()
        self.block_size = block_size
        self.intra_pos = nn.Parameter(torch.zeros(block_size, d_head))
        self.pool_logits = nn.Parameter(torch.zeros(block_size))
        self.proj = nn.Linear(d_head, d_head, bias=False)

    def forward(self, x_blocks):
        """``x_blocks [B,Hkv,n_blk,block_size,D] -> [B,Hkv,n_blk,D]``."""
        w = torch.softmax(self.pool_logits, dim=0)
        pooled = ((x_blocks + self.intra_pos) * w[:, None]).sum(dim=-2)
        return self.proj(pooled)


def _top_blocks(imp, k):
    """Top-k block indices per row, descending score then ascending index."""
    order = torch.sort(imp, dim=-1, descending=True, stable=True).indices
    return order[..., :k]


class NSAAttention(nn.Module):
    """NSA attention layer: shared query projection, per-branch key/value
    projections, learned compression poolers, per-head sigmoid gate over the
    three branches, output projection (nsa_model.py:130-195)."""

    def __init__(self, d_model, n_q_heads, n_kv_heads, block_size=16, n_selected_blocks=4, window=32,
                 attn_impl="ref"):
        super().__init__()
        assert n_q_heads % n_kv_heads == 0, "GQA needs n_q_heads divisible by n_kv_heads"
        assert attn_impl in ("ref", "fused"), "attn_impl must be 'ref' or 'fused'"
        self.d_model = d_model
        self.Hq = n_q_heads
        self.Hkv = n_kv_heads
        self.G = n_q_heads // n_kv_heads
        self.dh = d_model // n_q_heads
        self.block_size = block_size
        self.n_sel = n_selected_blocks
        self.window = window
        self.attn_impl = attn_impl
        self.register_buffer("scale", torch.tensor(self.dh ** -0.5), persistent=False)

        kv_dim = self.Hkv * self.dh
        self.q_proj = nn.Linear(d_model, self.Hq * self.dh, bias=False)
        self.k_cmp = nn.Linear(d_model, kv_dim, bias=False)
        self.v_cmp = nn.Linear(d_model, kv_dim, bias=False)
        self.k_slc = nn.Linear(d_model, kv_dim, bias=False)
        self.v_slc = nn.Linear(d_model, kv_dim, bias=False)
        self.k_win = nn.Linear(d_model, kv_dim, bias=False)
        self.v_win = nn.Linear(d_model, kv_dim, bias=False)
        self.comp_k = BlockCompressor(block_size, self.dh)
        self.comp_v = BlockCompressor(block_size, self.dh)
        self.gate = nn.Linear(d_model, self.Hq * 3, bias=True)
        self.out_proj = nn.Linear(self.Hq * self.dh, d_model, bias=False)

    # -- shared pieces ------------------------------------------------------
    def _heads(self, y, n_heads):
        B, T, _ = y.shape
        return y.view(B, T, n_heads, self.dh).transpose(1, 2)

    def _pooled(self, kc, vc, n_blk):
        B = kc.shape[0]
        L = self.block_size
        kb = kc[:, :, :n_blk * L].reshape(B, self.Hkv, n_blk, L, self.dh)
        vb = vc[:, :, :n_blk * L].reshape(B, self.Hkv, n_blk, L, self.dh)
        return self.comp_k(kb), self.comp_v(vb)

    def _gate_logits(self, x):
        B, T, _ = x.shape
        return self.gate(x).view(B, T, self.Hq, 3).permute(0, 2, 1, 3)      # [B,Hq,T,3]

    def _merge(self, out):
        B, _, T, _ = out.shape
        return self.out_proj(out.transpose(1, 2).reshape(B, T, self.Hq * self.dh))

    def forward(self, x, block_idx=None):
        if self.attn_impl == "fused":
            return self._forward_fused(x, block_idx)
        return self._forward_ref(x, block_idx)

    # -- dense torch definition (nsa_model.py:196-304) ------------------------
    def _forward_ref(self, x, block_idx=None):
        B, T, _ = x.shape
        L = self.block_size
        n_blk = T // L
        dev = x.device
        q = self._heads(self.q_proj(x), self.Hq)
        kc, vc = self._heads(self.k_cmp(x), self.Hkv), self._heads(self.v_cmp(x), self.Hkv)
        t = torch.arange(T, device=dev)

        o_cmp = q.new_zeros(q.shape)
        o_slc = q.new_zeros(q.shape)
        if n_blk > 0:
            k_cmp, v_cmp = self._pooled(kc, vc, n_blk)
            # pooled token j is visible once its whole block is in the past
            cmp_vis = (torch.arange(n_blk, device=dev) + 1) * L - 1 <= t[:, None]      # [T, n_blk]
            s_cmp = q @ expand_kv(k_cmp, self.G).transpose(-1, -2) * self.scale
            p_cmp = masked_softmax(s_cmp, cmp_vis.expand(B, self.Hq, T, n_blk))
            o_cmp = p_cmp @ expand_kv(v_cmp, self.G)

            # block choice: group-summed compression probabilities, detached
            imp = p_cmp.detach().view(B, self.Hkv, self.G, T, n_blk).sum(dim=2)
            imp = imp.masked_fill(~cmp_vis, torch.finfo(imp.dtype).min)
            if block_idx is None:
                sel = _top_blocks(imp, min(self.n_sel, n_blk))                     # [B,Hkv,T,S]
            else:
                sel = block_idx.to(device=dev, dtype=torch.long)
            self.last_block_idx = sel.to(torch.int32)
            hit = torch.zeros(B, self.Hkv, T, n_blk, dtype=torch.int32, device=dev)
            hit.scatter_add_(-1, sel.clamp(0, n_blk - 1), ((sel >= 0) & (sel < n_blk)).to(torch.int32))
            chosen = hit > 0
            blk_of_tok = (t // L).clamp(max=n_blk - 1)
            sel_keep = chosen[..., blk_of_tok] & (t[None, :] <= t[:, None]) & (t < n_blk * L)
            ks = expand_kv(self._heads(self.k_slc(x), self.Hkv), self.G)
            vs = expand_kv(self._heads(self.v_slc(x), self.Hkv), self.G)
            s_slc = q @ ks.transpose(-1, -2) * self.scale
            o_slc = masked_softmax(s_slc, expand_kv(sel_keep, self.G)) @ vs

        kw = expand_kv(self._heads(self.k_win(x), self.Hkv), self.G)
        vw = expand_kv(self._heads(self.v_win(x), self.Hkv), self.G)
        win_keep = (t[None, :] <= t[:, None]) & (t[:, None] - t[None, :] < self.window)
        s_win = q @ kw.transpose(-1, -2) * self.scale
        o_win = masked_softmax(s_win, win_keep.expand(B, self.Hq, T, T)) @ vw

        g = torch.sigmoid(self._gate_logits(x))
        out = g[..., 0:1] * o_cmp + g[..., 1:2] * o_slc + g[..., 2:3] * o_win
        return self._merge(out)

    # -- HIP kernels (nsa_model.py:306-370) -----------------------------------
    def _forward_fused(self, x, block_idx=None):
        import nsa_hip_ops as ops

        B, T, _ = x.shape
        L = self.block_size
        n_blk = T // L
        q = self._heads(self.q_proj(x), self.Hq).contiguous()
        kc, vc = self._heads(self.k_cmp(x), self.Hkv), self._heads(self.v_cmp(x), self.Hkv)
        if n_blk > 0:
            k_cmp, v_cmp = self._pooled(kc, vc, n_blk)
        else:
            k_cmp = q.new_zeros(B, self.Hkv, 0, self.dh)
            v_cmp = q.new_zeros(B, self.Hkv, 0, self.dh)
        ks = self._heads(self.k_slc(x), self.Hkv).contiguous()
        vs = self._heads(self.v_slc(x), self.Hkv).contiguous()
        kw = self._heads(self.k_win(x), self.Hkv).contiguous()
        vw = self._heads(self.v_win(x), self.Hkv).contiguous()
        gate_logits = self._gate_logits(x).contiguous()
        k_cmp, v_cmp, gate_logits = (y.to(q.dtype) for y in (k_cmp, v_cmp, gate_logits))
        geom = ops.NSAGeometry.aligned(L, self.n_sel, self.window)
        if block_idx is not None:
            block_idx = block_idx.to(device=q.device, dtype=torch.int32)
        out, block_idx = ops.nsa_attention(q, k_cmp.contiguous(), v_cmp.contiguous(), ks, vs, kw, vw,
                                           gate_logits, geom, block_idx=block_idx, pooled=True)
        self.last_block_idx = block_idx
        return self._merge(out)
