"""Window / compression branches, pooling and the gated three-branch NSA on
MI355X (drop-in for the reference module nsa_fused_kernel.py).

* ``_RangeAttn`` / ``window_attn_triton`` / ``compression_attn_triton`` keep
  the reference boundary (nsa_fused_kernel.py:521-543) on the HIP range
  kernels: a query-tiled forward (``nsa_range_fwd``), a query-side dQ kernel
  and a key-side dK/dV kernel.
* ``block_mean_pool`` (nsa_fused_kernel.py:549-554) is the HIP pooling kernel
  with its backward.
* ``nsa_fused_forward`` (nsa_fused_kernel.py:560-573) runs the whole gated
  three-branch layer inside one autograd boundary (``NSAFusedHIP``).
* ``nsa_attention`` adds what the reference leaves to the model: block choice
  by importance + top-n on the GPU and the overlapping compression /
  selection geometry (``NSAGeometry``).

``_range_attn_reference`` and ``nsa_fused_reference`` are the reference's
dense torch definitions (nsa_fused_kernel.py:576-609), kept for API parity;
the HIP path never calls them.
"""

import torch

import nsa_hip_ops as _ops
from nsa_hip_ops import NSAGeometry  # noqa: F401  (public)
from nsa_selection_kernel import selection_forward_reference
from nsa_selection_backward import selection_attn_hip

MODE_WINDOW = 0
MODE_COMPRESS = 1
USE_QTILE = True          # accepted and ignored: the HIP range kernels are always query-tiled

_RangeAttn = _ops.RangeAttnHIP


def window_attn_hip(q, k, v, window):
    return _RangeAttn.apply(q, k, v, MODE_WINDOW, window, 0)


def compression_attn_hip(q, k_cmp, v_cmp, block_size, cmp_stride=None):
    """Attention over pooled tokens; token i visible iff i*stride + block - 1 <= t."""
    return _RangeAttn.apply(q, k_cmp, v_cmp, MODE_COMPRESS, 0, block_size, cmp_stride)


window_attn_triton = window_attn_hip
compression_attn_triton = compression_attn_hip


def block_mean_pool(x, block_size, stride=None):
    """[B,H,T,D] -> [B,H,n,D] mean over [i*stride, i*stride + block_size)."""
    return _ops.pool_mean(x, block_size, block_size if stride is None else stride)


def nsa_fused_forward(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, block_size, window):
    """Full NSA attention output (pre out_proj) on the HIP path, aligned grid.

    q [B,Hq,T,D]; kc/vc/ks/vs/kw/vw [B,Hkv,T,D]; gate_logits [B,Hq,T,3];
    block_idx [B,Hkv,T,S] (non-differentiable selection input).
    """
    S = block_idx.shape[-1]
    geom = NSAGeometry.aligned(block_size, S, window)
    out, _ = _ops.NSAFusedHIP.apply(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, geom)
    return out


def nsa_attention(q, kc, vc, ks, vs, kw, vw, gate_logits, geom, block_idx=None):
    """NSA attention with an explicit geometry; ``(out, block_idx)``.

    ``block_idx=None`` selects blocks on the GPU from the compression
    importance (ties to the lower block index).
    """
    return _ops.nsa_attention(q, kc, vc, ks, vs, kw, vw, gate_logits, geom, block_idx)


def nsa_fused_forward_composed(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, block_size, window):
    """The reference's composition (pool, three per-branch Functions, torch gate)
    on the HIP branch kernels; same result as ``nsa_fused_forward``."""
    k_cmp = block_mean_pool(kc, block_size)
    v_cmp = block_mean_pool(vc, block_size)
    o_cmp = compression_attn_hip(q, k_cmp, v_cmp, block_size)
    o_slc = selection_attn_hip(q, ks, vs, block_idx, block_size)
    o_win = window_attn_hip(q, kw, vw, window)
    g = torch.sigmoid(gate_logits)
    return g[..., 0:1] * o_cmp + g[..., 1:2] * o_slc + g[..., 2:3] * o_win


# ---------------------------------------------------------------------------
# the reference's dense definitions (torch, any device)
# ---------------------------------------------------------------------------

def _range_attn_reference(q, k, v, mode, window, block_size):
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    Lk = k.shape[2]
    scale = D ** -0.5
    kexp = k.float().repeat_interleave(G, dim=1)
    vexp = v.float().repeat_interleave(G, dim=1)
    s = torch.matmul(q.float(), kexp.transpose(-1, -2)) * scale
    tt = torch.arange(T, device=q.device)[:, None]
    jj = torch.arange(Lk, device=q.device)[None, :]
    if mode == MODE_WINDOW:
        keep = (jj <= tt) & (tt - jj < window)
    else:
        keep = (jj + 1) * block_size - 1 <= tt
    keep = keep[None, None].expand(B, Hq, T, Lk)
    s = s.masked_fill(~keep, torch.finfo(s.dtype).min)
    p = torch.softmax(s, dim=-1) * keep.any(dim=-1, keepdim=True)
    return torch.matmul(p, vexp).to(q.dtype)


def _block_mean_pool_torch(x, block_size):
    B, H, T, D = x.shape
    n = T // block_size
    return x[:, :, :n * block_size].reshape(B, H, n, block_size, D).mean(dim=3)


def nsa_fused_reference(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, block_size, window):
    k_cmp = _block_mean_pool_torch(kc, block_size)
    v_cmp = _block_mean_pool_torch(vc, block_size)
    o_cmp = _range_attn_reference(q, k_cmp, v_cmp, MODE_COMPRESS, 0, block_size)
    o_slc = selection_forward_reference(q, ks, vs, block_idx, block_size)
    o_win = _range_attn_reference(q, kw, vw, MODE_WINDOW, window, 0)
    g = torch.sigmoid(gate_logits)
    return g[..., 0:1] * o_cmp + g[..., 1:2] * o_slc + g[..., 2:3] * o_win
