"""The whole gated layer through its two C entry points (nsa_fused_fwd /
nsa_fused_bwd, include/nsa_hip.h) against the Python autograd boundary
(NSAFusedHIP) on the same inputs: the same launches in the same order, so the
output, the block indices and all eight gradients are bit-identical -- GQA
groups of 16 and 6 heads, bf16 and float32, block choice made in the call or
given, pooled compression tokens from the caller, and the aligned reference
grid."""

import pytest
import torch

from nsa_testlib import log, randn, require_gpu

pytestmark = pytest.mark.gpu

BASE = (32, 16, 64, 16, 512, False, 0)

CASES = [
    ("g16-d128-bf16", 1, 16, 1, 2048, 128, torch.bfloat16, BASE, False, False),
    ("g6-d64-bf16-forced", 2, 12, 2, 1536, 64, torch.bfloat16, (32, 16, 64, 8, 256, True, 2), False, False),
    ("g4-d64-f32", 1, 8, 2, 1024, 64, torch.float32, (32, 16, 64, 8, 128, False, 0), False, False),
    ("g16-d128-bf16-idx-given", 1, 16, 1, 1024, 128, torch.bfloat16, BASE, True, False),
    ("g6-d64-bf16-pooled", 1, 12, 2, 1024, 64, torch.bfloat16, BASE, False, True),
    ("g4-d32-aligned64", 1, 16, 4, 1024, 32, torch.bfloat16, (64, 64, 64, 8, 200, False, 0), False, False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_capi_equals_the_python_boundary(case):
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    name, B, Hq, Hkv, T, D, dtype, gp, idx_given, pooled = case
    geom = ops.NSAGeometry(*gp)
    n = ops.n_cmp_tokens(T, geom.cmp_block, geom.cmp_stride)
    Tc = n if pooled else T
    ins = [randn((B, Hq, T, D), 1, dtype)] + [randn((B, Hkv, Tc if i < 2 else T, D), 2 + i, dtype)
                                              for i in range(6)] + [randn((B, Hq, T, 3), 9, dtype)]
    ins = [t.to(dev) for t in ins]
    do = randn((B, Hq, T, D), 10, dtype).to(dev)
    idx0 = None
    if idx_given:
        _, idx0 = nfk.nsa_attention(*ins, geom)
        idx0 = torch.flip(idx0, dims=[-1]).contiguous()   # another order of the same blocks
    xs = [t.clone().requires_grad_() for t in ins]
    out, idx = ops.NSAFusedHIP.apply(*xs, idx0, geom, pooled)
    out.backward(do)
    out_c, idx_c, grads_c = ops.fused_capi(*ins, geom, do, block_idx=idx0, pooled=pooled)
    torch.cuda.synchronize()
    assert torch.equal(idx_c, idx), f"{name}: block indices differ"
    assert torch.equal(out_c, out.detach()), f"{name}: output differs"
    for nm, g, x in zip(["q", "kc", "vc", "ks", "vs", "kw", "vw", "gate"], grads_c, xs):
        assert torch.equal(g, x.grad), f"{name}: d{nm} differs (max {float((g - x.grad).abs().max()):.3e})"
        assert float(g.abs().max()) > 0, f"{name}: d{nm} all zero"
    log(f"  {name}: out, indices and 8 gradients bit-identical to the Python boundary")


@pytest.mark.parametrize("case", [CASES[1], CASES[4]], ids=[CASES[1][0], CASES[4][0]])
def test_capi_autograd_equals_the_python_boundary(case):
    """NSAFusedCAPI (the model layer's path: one C call per direction, the
    context saved between them, scratch per call) against NSAFusedHIP under
    autograd, twice in a row (the second call reuses the first's freed
    buffers)."""
    dev = require_gpu()
    import nsa_hip_ops as ops
    name, B, Hq, Hkv, T, D, dtype, gp, _, pooled = case
    geom = ops.NSAGeometry(*gp)
    n = ops.n_cmp_tokens(T, geom.cmp_block, geom.cmp_stride)
    Tc = n if pooled else T
    for rep in range(2):
        ins = [randn((B, Hq, T, D), 1 + rep, dtype)] + [randn((B, Hkv, Tc if i < 2 else T, D), 2 + i + rep, dtype)
                                                        for i in range(6)] + [randn((B, Hq, T, 3), 9 + rep, dtype)]
        ins = [t.to(dev) for t in ins]
        do = randn((B, Hq, T, D), 10 + rep, dtype).to(dev)
        xs = [t.clone().requires_grad_() for t in ins]
        ys = [t.clone().requires_grad_() for t in ins]
        out, idx = ops.NSAFusedHIP.apply(*xs, None, geom, pooled)
        out.backward(do)
        out_c, idx_c = ops.NSAFusedCAPI.apply(*ys, None, geom, pooled)
        out_c.backward(do)
        torch.cuda.synchronize()
        assert torch.equal(idx_c, idx) and torch.equal(out_c, out), f"{name}: forward differs"
        for nm, x, y in zip(["q", "kc", "vc", "ks", "vs", "kw", "vw", "gate"], xs, ys):
            assert torch.equal(y.grad, x.grad), f"{name}: d{nm} differs"
    log(f"  {name}: the C-ABI autograd path bit-identical, two calls")


def test_fused_capi_rejects_bad_calls():
    require_gpu()
    import _nsa_lib as L
    lib = L.load()
    # T below the selection block: no size (the layer needs both branches' blocks)
    assert lib.nsa_fused_ctx_bytes(1, 16, 1, 48, 128, 32, 16, 64, 16, 512, 0, 1) == 0
    # too small a scratch buffer: rejected before any launch
    fake = 1 << 20
    ctx = lib.nsa_fused_ctx_bytes(1, 16, 1, 1024, 128, 32, 16, 64, 16, 512, 0, 1)
    rc = lib.nsa_fused_fwd(*([fake] * 8), fake, 0, fake, fake, ctx, fake, 256, 1, 16, 1, 1024, 128, 32, 16, 64, 16,
                           512, 0, 0, 0, 1, None)
    assert rc == L.NSA_ERR_WORKSPACE
