"""nsa_sel_dkdv_noalloc -- the selection dK/dV with its work-item list in
the library's fixed device array -- against nsa_sel_dkdv with a caller
workspace, through the C-ABI, on two calls in a row (the second smaller, so
it runs over the first call's leftovers in the array).

dQ partials (of the slots that have a causal pair; the others are never
written) are plain stores of identical kernels: bit-exact.  dK / dV merge
work-item partials with float atomics, whose order can differ: float32
inputs, within 1e-5 relative to the largest value (the fp32 parity bar is
1e-4).
"""

import ctypes

import pytest
import torch

from nsa_testlib import log, make_block_idx, randn, require_gpu

pytestmark = pytest.mark.gpu

CASES = [  # (B, Hq, Hkv, T, D, block_size, S): each call smaller than the one before
    (2, 16, 2, 2048, 64, 64, 8),   # G = 8: group-packed row tiles
    (1, 8, 1, 512, 32, 32, 4),
    (1, 16, 1, 384, 32, 32, 4),    # G = 16: two queries x 16 heads per tile
]


def _run_case(dev, B, Hq, Hkv, T, D, bs, S, seed):
    import _nsa_lib as L
    import nsa_hip_ops as ops
    dtype = torch.float32
    q = randn((B, Hq, T, D), seed + 1, dtype).to(dev)
    k = randn((B, Hkv, T, D), seed + 2, dtype).to(dev)
    v = randn((B, Hkv, T, D), seed + 3, dtype).to(dev)
    do = randn((B, Hq, T, D), seed + 4, dtype).to(dev)
    idx = make_block_idx(B, Hkv, T, bs, S, seed=seed).to(dev)
    o, lse = ops.sel_fwd(q, k, v, idx, bs)
    # row statistics in the packed row order [B, Hkv, T, G], dO packed
    dot, coff, dop = ops.delta_of(do, o, lse, pack_hkv=Hkv)
    qp = ops.pack_heads(q, Hkv)
    kt = ops.transpose_kv(k)
    csr = ops.csr_device(idx, bs, pack_slot=True)
    chunk = ops.SEL_DKDV_CHUNK
    # caller-workspace entry point
    dk_ref, dv_ref, dq_ref = ops.sel_dkdv(q, k, v, do, coff, dot, idx, bs, csr=csr, kt=kt, want_dq=True,
                                          qp=qp, dop=dop, stats_packed=True)
    # no-alloc entry point: outputs allocated here, nothing inside the call
    dk = torch.full_like(dk_ref, float("nan"))
    dv = torch.full_like(dv_ref, float("nan"))
    dq = torch.full_like(dq_ref, float("nan"))
    q_of_block, offsets, _, count = csr
    lib = L.load()
    rc = lib.nsa_sel_dkdv_noalloc(L.ptr(qp), L.ptr(k), L.ptr(v), L.ptr(kt), L.ptr(dop), L.ptr(coff), L.ptr(dot),
                                  L.ptr(q_of_block), 1, L.ptr(offsets), L.ptr(count), L.ptr(dk), L.ptr(dv),
                                  L.ptr(dq), B, Hq, Hkv, T, D, S, bs, chunk, L.dtype_code(q),
                                  ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert rc == 0, f"nsa_sel_dkdv_noalloc returned {rc}"
    torch.cuda.synchronize()
    # partials exist for the slots with a causal pair only (the others are
    # never written): j >= 0 and j * block_size <= t, one pass per 64 keys
    npass = -(-bs // 64)
    t = torch.arange(T, device=dev)[None, None, :, None]
    valid = ((idx >= 0) & (idx.long() * bs <= t)).repeat_interleave(npass, dim=-1)
    assert dq.shape[3] == S * npass
    assert torch.equal(dq[valid], dq_ref[valid]), "dQ partials differ"
    assert int(valid.sum()) > 0
    for nm, a, b in (("dk", dk, dk_ref), ("dv", dv, dv_ref)):
        err = float((a - b).abs().max())
        ref = float(b.abs().max())
        log(f"  {nm}: max_abs {err:.3e} (|ref|max {ref:.3e})")
        assert err <= 1e-5 * max(1.0, ref), f"{nm}: {err:.3e}"


def test_sel_dkdv_noalloc_matches_workspace_entry_point():
    dev = require_gpu()
    for i, c in enumerate(CASES):
        log(f"no-alloc selection dK/dV, call {i + 1}: B{c[0]} Hq{c[1]} Hkv{c[2]} T{c[3]} D{c[4]} bs{c[5]} S{c[6]}")
        _run_case(dev, *c, seed=10 * i)


def test_sel_dkdv_noalloc_rejects_oversize():
    import _nsa_lib as L
    lib = L.load()
    # chunk 2 at this size needs far more work items than the array holds:
    # refused before anything touches the device
    rc = lib.nsa_sel_dkdv_noalloc(*([None] * 8), 1, *([None] * 5), 1, 16, 1, 65536, 64, 16, 64, 2, 1, None)
    assert rc == L.NSA_ERR_WORKSPACE
