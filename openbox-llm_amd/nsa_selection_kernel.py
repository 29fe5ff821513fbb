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

``selection_forward_reference`` is a dense torch definition of
the branch (nsa_selection_kernel.py:55-92), kept for API parity; the HIP path
never calls it.
"""

import torch

import nsa_hip_ops as _ops

USE_FSA_FWD = True


def dense_branch_attention(q, k, v, keep):
    """Softmax attention of ``q [B,Hq,T,D]`` over ``k/v [B,Hkv,L,D]``
    restricted to ``keep`` (bool, broadcastable to ``[B,Hkv,T,L]``): float32
    math, output in q's dtype, rows with no kept key zero.  Built on
    ``nsa_model.masked_softmax`` / ``expand_kv``; the dense definitions of
    the three branches are this function with their masks."""
    from nsa_model import expand_kv, masked_softmax
    B, Hq, T, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    keep = expand_kv(torch.as_tensor(keep, device=q.device).expand(B, Hkv, T, L), G)
    scores = torch.matmul(q.float(), expand_kv(k.float(), G).transpose(-1, -2).contiguous()) * D ** -0.5
    return (masked_softmax(scores, keep) @ expand_kv(v.float(), G)).to(q.dtype)


def selection_keep(block_idx, T, block_size):
    """``[B,Hkv,T,T]`` mask of the selection branch: key p is kept for query
    t iff its block ``p // block_size`` is listed in ``block_idx[..., t, :]``
    (-1 = empty slot) and p <= t; a trailing partial block is reached like any
    other (nsa_selection_kernel.py:74-85)."""
    B, Hkv, _, S = block_idx.shape
    dev = block_idx.device
    n_blk = -(-T // block_size)
    idx = block_idx.long()
    listed = torch.zeros(B, Hkv, T, n_blk + 1, dtype=torch.bool, device=dev)
    # empty or out-of-range slots land in the spare last column, which no key reads
    listed.scatter_(-1, torch.where((idx >= 0) & (idx < n_blk), idx, torch.full_like(idx, n_blk)), True)
    pos = torch.arange(T, device=dev)
    return listed[..., pos // block_size] & (pos[None, :] <= pos[:, None])


def selection_forward_reference(q, k, v, block_idx, block_size):
    """Dense masked selection attention, float32 math, output in q's dtype
    (the definition of nsa_selection_kernel.py:55-92)."""
    return dense_branch_attention(q, k, v, selection_keep(block_idx, q.shape[2], block_size))


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
