"""The block-outer selection kernels (nsa_sel_fwd_bo, nsa_sel_dkdv) on a CSR
whose entries do NOT ascend within a block: every block's entries reversed.
The kernels address a tile's two query rows upward from the lower one
(pair_rows), so the reversed order reads the same rows: the forward partials
and dQ partials of every (query, slot) are bit-exact against the ascending
CSR; dK / dV agree up to the fp32 summation order of the tiles (1e-4 of
their largest magnitude).  (Regression of an out-of-bounds
read: both offsets were taken from query A, which wrapped when B < A.)
"""

import pytest
import torch

from nsa_testlib import log, make_block_idx, randn, require_gpu

pytestmark = pytest.mark.gpu


def _reversed_blocks(q_of_block, offsets):
    """The CSR entries of every block in reverse order (same pairs)."""
    rev = q_of_block.clone()
    off = offsets.view(-1).tolist()
    for a, e in zip(off[:-1], off[1:]):
        if e > a:
            rev[a:e] = q_of_block[a:e].flip(0)
    return rev


@pytest.mark.parametrize("heads", [(16, 1), (12, 2)], ids=["G16", "G6"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_unsorted_csr_matches_sorted(dtype, heads):
    """G16: two queries per row tile; G6: five entries per tile, so the
    reversal also changes which entries share a tile."""
    import nsa_hip_ops as ops
    dev = require_gpu()
    B, Hq, Hkv, T, D, bs, S = 1, heads[0], heads[1], 1024, 64, 64, 8
    log(f"csr order: B{B} Hq{Hq} Hkv{Hkv} T{T} D{D} bs{bs} S{S} {dtype}")
    q = randn((B, Hq, T, D), 1, dtype).to(dev)
    k = randn((B, Hkv, T, D), 2, dtype).to(dev)
    v = randn((B, Hkv, T, D), 3, dtype).to(dev)
    do = randn((B, Hq, T, D), 4, dtype).to(dev)
    idx = make_block_idx(B, Hkv, T, bs, S, seed=5).to(dev)
    csr = ops.csr_device(idx, bs, pack_slot=True)
    qob, off, pbh, cnt = csr
    # one block's entries hold one pair per (query, slot): offsets are per (bh, block) over B*Hkv rows of n_blk+1
    n_blk = off.shape[-1] - 1
    rows = off.view(-1, n_blk + 1)
    rev = qob.clone()
    for r in range(rows.shape[0]):
        rev_r = _reversed_blocks(qob, rows[r])
        lo, hi = int(rows[r][0]), int(rows[r][-1])
        rev[lo:hi] = rev_r[lo:hi]
    assert not torch.equal(rev[:int(cnt.item())], qob[:int(cnt.item())]), "the reversal must change the order"
    csr_rev = (rev, off, pbh, cnt)
    t = torch.arange(T, device=dev)[None, None, :, None]
    valid = (idx >= 0) & (idx.long() * bs <= t)   # slots with a causal pair (one pass per 64 keys)

    (o1, m1), _ = ops.sel_fwd_partials(q, k, v, idx, bs, csr=csr)
    (o2, m2), _ = ops.sel_fwd_partials(q, k, v, idx, bs, csr=csr_rev)
    torch.cuda.synchronize()
    assert torch.equal(o1[valid], o2[valid]) and torch.equal(m1[valid], m2[valid]), "forward partials differ"

    o, lse = ops.sel_fwd(q, k, v, idx, bs)
    dot, coff, dop = ops.delta_of(do, o, lse, pack_hkv=Hkv)
    qp = ops.pack_heads(q, Hkv)
    kt = ops.transpose_kv(k)
    r1 = ops.sel_dkdv(q, k, v, do, coff, dot, idx, bs, csr=csr, kt=kt, want_dq=True, qp=qp, dop=dop,
                      stats_packed=True)
    r2 = ops.sel_dkdv(q, k, v, do, coff, dot, idx, bs, csr=csr_rev, kt=kt, want_dq=True, qp=qp, dop=dop,
                      stats_packed=True)
    torch.cuda.synchronize()
    assert torch.equal(r1[2][valid], r2[2][valid]), "dQ partials differ"
    for nm, a, b in (("dk", r1[0], r2[0]), ("dv", r1[1], r2[1])):
        err = float((a - b).abs().max())
        ref = float(b.abs().max())
        log(f"  {nm}: max_abs {err:.3e} (|ref|max {ref:.3e})")
        assert err <= 1e-4 * max(1.0, ref), f"{nm}: {err:.3e}"
