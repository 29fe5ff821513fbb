"""Block -> query CSR on MI355X (drop-in for the reference module nsa_fsa.py).

``build_block_to_query_csr`` keeps the reference contract (nsa_fsa.py:14-64):
pairs (t, j) with j >= 0 and j*block_size <= t, grouped by (b, hkv, block)
with queries ascending, global offsets.  It runs as a counting build on the
GPU (``nsa_csr_build``: per-(block, query chunk) counts, an exclusive scan,
then placement in query order; a radix sort only past the counting build's LDS
budget); the exact pair count is read back once to size the returned tensors,
as the reference's ``nonzero`` does.
"""

import torch

import nsa_hip_ops as _ops


@torch.no_grad()
def build_block_to_query_csr(block_idx, block_size):
    """-> (q_of_block [P], block_offsets [B,Hkv,n_blk+1], pair_bh [P]), int32.

    ``n_blk = T // block_size`` as in the reference (nsa_fsa.py:36).  A causal
    pair whose block lies past that grid (the trailing partial block) has no
    row in the reference's CSR and makes its ``scatter_add_`` fail
    (nsa_fsa.py:46-48); here it raises IndexError.
    """
    assert block_idx.is_cuda, "block_idx must be a GPU tensor"
    B, Hkv, T, S = block_idx.shape
    n_blk = T // block_size
    t = torch.arange(T, device=block_idx.device, dtype=torch.int64)[:, None]
    idx = block_idx.to(torch.int64)
    if bool(((idx >= n_blk) & (idx * block_size <= t)).any()):
        raise IndexError(f"block index >= T // block_size = {n_blk} on a causal pair")
    q_of_block, offsets, pair_bh, count = _ops.csr_device(block_idx, block_size, n_blk)
    P = int(count.item())
    return q_of_block[:P].contiguous(), offsets, pair_bh[:P].contiguous()
