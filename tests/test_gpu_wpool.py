"""GPU parity of the learned weighted pool (nsa_wpool_fwd / _bwd / _dw
behind nsa_hip_ops.weighted_pool and BlockCompressor.pool_sequence) against
the module's own unfolded form (BlockCompressor.forward, nsa_model.py:100-123)
in float64 on the CPU: the pooled tokens after the projection and the
gradients of x, pool_logits, intra_pos and the projection weight."""

import pytest
import torch

from nsa_testlib import assert_close, log, require_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("geo", [(32, 16, 300, 64), (16, 16, 256, 128), (48, 16, 333, 32), (32, 8, 97, 16),
                                 (32, 16, 20, 64)],
                         ids=["l2d", "l=d", "l3d-ragged", "l4d-D16", "no-span"])
def test_weighted_pool_matches_unfolded_module(geo, dtype):
    import nsa_model
    dev = require_gpu()
    l, d, T, D = geo
    log(f"weighted pool l{l} d{d} T{T} D{D} {dtype}")
    torch.manual_seed(0)
    comp = nsa_model.BlockCompressor(l, D)
    with torch.no_grad():
        comp.pool_logits.normal_()
        comp.intra_pos.normal_()
        comp.proj.weight.mul_(4.0)
    B, H = 2, 3
    x = torch.randn(B, H, T, D).to(dtype)
    n = (T - l) // d + 1 if T >= l else 0
    cot = torch.randn(B, H, max(n, 0), D, dtype=torch.float64)
    if n == 0:
        # shorter than one span: no pooled token, zero gradients
        xg = x.to(dev).requires_grad_()
        got = comp.to(dev).pool_sequence(xg, d)
        got.sum().backward()
        torch.cuda.synchronize()
        assert got.shape == (B, H, 0, D)
        assert float(xg.grad.abs().max()) == 0.0
        assert float(comp.pool_logits.grad.abs().max()) == 0.0
        return
    # reference: the unfolded module in float64
    ref_mod = nsa_model.BlockCompressor(l, D).double()
    ref_mod.load_state_dict({k: v.double() for k, v in comp.state_dict().items()})
    xr = x.double().requires_grad_()
    blocks = xr[:, :, :max((n - 1) * d + l, 0)].unfold(2, l, d).transpose(-1, -2)
    ref = ref_mod(blocks)
    (ref * cot).sum().backward()
    # HIP: the module's parameters in float32, x in dtype (as under autocast)
    mod = comp.to(dev)
    xg = x.to(dev).requires_grad_()
    got = mod.pool_sequence(xg, d)
    (got.double() * cot.to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert got.shape == ref.shape
    assert_close(got.float().cpu(), ref, torch.float32, "pooled")
    assert_close(xg.grad.float().cpu(), xr.grad, dtype, "dx")
    for name in ("pool_logits", "intra_pos", "proj.weight"):
        g = dict(mod.named_parameters())[name].grad.cpu()
        r = dict(ref_mod.named_parameters())[name].grad
        assert_close(g, r, torch.float32, f"d{name}")
