"""Selection-branch backward and its autograd boundary on MI355X (drop-in for
the reference module nsa_selection_backward.py).

Gradients (nsa_selection_backward.py:12-20): delta = dO.O, dS = P (dP - delta),
dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO.  dK/dV always come from a
block-outer kernel over the block -> query CSR built on the GPU
(``nsa_csr_build`` + ``nsa_sel_dkdv``).  ``selection_backward_triton`` takes dQ
from a query-outer kernel (``nsa_sel_dq``); ``selection_backward_fsa`` and the
autograd boundary take it from the block-outer kernel as per-(query, block)
partials in the input dtype, summed by ``nsa_sel_dq_reduce``.
``USE_FSA_BWD`` is accepted and ignored.
"""

import nsa_hip_ops as _ops
from nsa_selection_kernel import selection_forward_hip  # noqa: F401  (reference import surface)

USE_FSA_BWD = True


def selection_backward_hip(q, k, v, block_idx, block_size, do, o):
    """(dq, dk, dv) in the input dtypes; recomputes the softmax statistics."""
    return _ops.selection_backward(q, k, v, block_idx, block_size, do, o)


def selection_backward_fsa(q, k, v, block_idx, block_size, do, o, lse):
    """(dq, dk, dv) using the stored lse of the forward, block-outer: one
    kernel writes dK/dV and per-(query, block) dQ partials, a reduce sums them."""
    return _ops.selection_backward_fsa(q, k, v, block_idx, block_size, do, o, lse)


selection_backward_triton = selection_backward_hip

SelectionAttnHIP = _ops.SelectionAttnHIP
SelectionAttnTriton = SelectionAttnHIP


def selection_attn_hip(q, k, v, block_idx, block_size):
    return SelectionAttnHIP.apply(q, k, v, block_idx, block_size)


selection_attn_triton = selection_attn_hip
