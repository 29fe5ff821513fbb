"""Selection-branch backward and its autograd boundary on MI355X (drop-in for
the reference module nsa_selection_backward.py).

Gradients (nsa_selection_backward.py:12-20): delta = dO.O, dS = P (dP - delta),
dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO.  dQ comes from a query-outer
HIP kernel (``nsa_sel_dq``, registers only); dK/dV from a block-outer kernel
over the block -> query CSR built on the GPU (``nsa_csr_build`` +
``nsa_sel_dkdv``), so no per-pair partial buffers are materialised.
``USE_FSA_BWD`` is accepted and ignored (one path serves every shape).
"""

import nsa_hip_ops as _ops
from nsa_selection_kernel import selection_forward_hip  # noqa: F401  (reference import surface)

USE_FSA_BWD = True


def selection_backward_hip(q, k, v, block_idx, block_size, do, o):
    """(dq, dk, dv) in the input dtypes; recomputes the softmax statistics."""
    return _ops.selection_backward(q, k, v, block_idx, block_size, do, o)


def selection_backward_fsa(q, k, v, block_idx, block_size, do, o, lse):
    """(dq, dk, dv) using the stored lse of the forward."""
    return _ops.selection_backward(q, k, v, block_idx, block_size, do, o, lse)


selection_backward_triton = selection_backward_hip

SelectionAttnHIP = _ops.SelectionAttnHIP
SelectionAttnTriton = SelectionAttnHIP


def selection_attn_hip(q, k, v, block_idx, block_size):
    return SelectionAttnHIP.apply(q, k, v, block_idx, block_size)


selection_attn_triton = selection_attn_hip
