"""Selection-branch forward on MI355X (drop-in for the reference module
nsa_selection_kernel.py).

``selection_forward_triton`` / ``selection_forward_fsa`` keep their names and
return conventions (nsa_selection_kernel.py:175-213, :294-365) on HIP
kernels.  ``selection_forward_triton`` is query-outer (``nsa_sel_fwd``: one
wave per query and 16-head column block, the selected blocks gathered 32 keys
per MFMA step).  ``selection_forward_fsa`` is block-outer (``nsa_sel_fwd_bo``:
one wave holds a selected block's keys and streams the queries that chose
it, writing per-(query, block) partials that ``nsa_sel_merge`` combines).  The
module switch ``USE_FSA_FWD`` is accepted and ignored: the autograd boundary
always runs block-outer.

``selection_forward_reference`` is the reference's dense torch definition of
the branch (nsa_selection_kernel.py:55-92), kept for API parity; the HIP path
never calls it.
"""

import torch

import nsa_hip_ops as _ops

USE_FSA_FWD = True


def selection_forward_reference(q, k, v, block_idx, block_size):
    """Dense masked selection attention (float32 math, output in q's dtype)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    dev = q.device
    scale = D ** -0.5
    qf = q.float()
    kexp = k.float().repeat_interleave(G, dim=1)
    vexp = v.float().repeat_interleave(G, dim=1)
    s = torch.matmul(qf, kexp.transpose(-1, -2)) * scale
    p_idx = torch.arange(T, device=dev)
    blk_of_p = p_idx // block_size
    idx = block_idx.long()
    chosen = ((idx[..., :, None] == blk_of_p) & (idx[..., :, None] >= 0)).any(dim=3)   # [B,Hkv,T,T]
    keep = chosen & (p_idx[None, :] <= p_idx[:, None])[None, None]
    keep = keep.repeat_interleave(G, dim=1)
    s = s.masked_fill(~keep, torch.finfo(s.dtype).min)
    p = torch.softmax(s, dim=-1) * keep.any(dim=-1, keepdim=True)
    return torch.matmul(p, vexp).to(q.dtype)


def selection_forward_hip(q, k, v, block_idx, block_size, return_lse=False):
    """q [B,Hq,T,D], k/v [B,Hkv,T,D], block_idx [B,Hkv,T,S] -> o (, lse)."""
    o, lse = _ops.sel_fwd(q, k, v, block_idx, block_size)
    return (o, lse) if return_lse else o


def selection_forward_fsa(q, k, v, block_idx, block_size):
    """Block-outer forward over the block -> query CSR: (o, lse), as the
    reference's FSA path (nsa_selection_kernel.py:294-365)."""
    o, lse, _ = _ops.sel_fwd_fsa(q, k, v, block_idx, block_size)
    return o, lse


selection_forward_triton = selection_forward_hip
