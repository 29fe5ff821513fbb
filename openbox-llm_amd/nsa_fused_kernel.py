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

``_range_attn_reference`` and ``nsa_fused_reference`` are dense torch
definitions of the same functions (nsa_fused_kernel.py:576-609), kept for
API parity; the HIP path never calls them.
"""

import torch

import nsa_hip_ops as _ops
from nsa_hip_ops import NSAGeometry  # noqa: F401  (public)
from nsa_selection_kernel import dense_branch_attention, selection_forward_reference
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
# dense definitions (torch, any device): the branches' masks on one helper
# ---------------------------------------------------------------------------

def _range_attn_reference(q, k, v, mode, window, block_size):
    """Dense window (mode 0: keys t - window < p <= t) or compression (mode 1:
    pooled token j once ``(j + 1) * block_size - 1 <= t``) attention, float32
    math, output in q's dtype (nsa_fused_kernel.py:576-597)."""
    t = torch.arange(q.shape[2], device=q.device)[:, None]
    j = torch.arange(k.shape[2], device=q.device)[None, :]
    keep = ((j <= t) & (t - j < window)) if mode == MODE_WINDOW else ((j + 1) * block_size - 1 <= t)
    return dense_branch_attention(q, k, v, keep)


def _block_mean_pool_torch(x, block_size):
    """Mean over the complete non-overlapping blocks of the sequence axis."""
    return x.unfold(2, block_size, block_size).mean(dim=-1)


def nsa_fused_reference(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, block_size, window):
    """The gated three-branch output from the dense definitions
    (nsa_fused_kernel.py:600-609)."""
    o = [_range_attn_reference(q, _block_mean_pool_torch(kc, block_size), _block_mean_pool_torch(vc, block_size),
                               MODE_COMPRESS, 0, block_size),
         selection_forward_reference(q, ks, vs, block_idx, block_size),
         _range_attn_reference(q, kw, vw, MODE_WINDOW, window, 0)]
    g = torch.sigmoid(gate_logits)
    return sum(g[..., c:c + 1] * o[c] for c in range(3))
