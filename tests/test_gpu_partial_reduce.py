"""The selection dQ partial reduce (nsa_sel_dq_reduce through
nsa_hip_ops.sel_dq_reduce): the sum of every row's valid-slot partials,
rounded once to the partials' dtype, and a float32 request is that result
converted -- the kernel always reads the partials as the type they are
stored in.  (Regression: a float32 request on bf16 partials used to hand the
bf16 buffer to the reduce as float32, which read past its end.)"""

import pytest
import torch

from nsa_testlib import log, make_block_idx, randn, require_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("heads", [(16, 1), (12, 2)], ids=["G16", "G6"])
def test_dq_reduce_sums_valid_slots_in_the_partials_dtype(heads):
    import nsa_hip_ops as ops
    dev = require_gpu()
    B, Hq, Hkv, T, D, bs, S = 1, heads[0], heads[1], 1024, 64, 64, 8
    G = Hq // Hkv
    log(f"dq reduce: B{B} Hq{Hq} Hkv{Hkv} T{T} D{D} bs{bs} S{S} bf16")
    q = randn((B, Hq, T, D), 11, torch.bfloat16).to(dev)
    k = randn((B, Hkv, T, D), 12, torch.bfloat16).to(dev)
    v = randn((B, Hkv, T, D), 13, torch.bfloat16).to(dev)
    do = randn((B, Hq, T, D), 14, torch.bfloat16).to(dev)
    idx = make_block_idx(B, Hkv, T, bs, S, seed=15).to(dev)
    o, lse = ops.sel_fwd(q, k, v, idx, bs)
    dot, coff = ops.delta_of(do, o, lse)
    _, _, part = ops.sel_dkdv(q, k, v, do, coff, dot, idx, bs, want_dq=True)
    r16 = ops.sel_dq_reduce(idx, part, None, bs, torch.bfloat16)
    r32 = ops.sel_dq_reduce(idx, part, None, bs, torch.float32)
    torch.cuda.synchronize()
    assert part.dtype == torch.bfloat16 and r16.dtype == torch.bfloat16 and r32.dtype == torch.float32
    assert torch.equal(r32, r16.float()), "the float32 request is not the reduce's result converted"
    # the valid slots (a block that starts at or before the query) summed in
    # float32; the partials of the other slots are never written (selected,
    # not multiplied by 0: their bytes may be anything)
    t = torch.arange(T, device=dev)[None, None, :, None]
    valid = (idx >= 0) & (idx.long() * bs <= t)                                # [B, Hkv, T, S]
    ns = part.shape[3]
    assert ns == S, "one pass per slot at block size 64"
    ref = torch.where(valid[..., None, None], part.float(), 0.0).sum(3)         # [B, Hkv, T, G, D]
    ref = ref.permute(0, 1, 3, 2, 4).reshape(B, Hq, T, D)
    err = float(((r32 - ref).abs() / ref.abs().clamp_min(1.0)).max())
    log(f"  reduce vs float32 sum of the valid partials: {err:.2e}")
    assert err <= 2.0 ** -8, f"reduce differs from the partial sum ({err:.2e})"
