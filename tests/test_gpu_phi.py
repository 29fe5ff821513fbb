"""GPU parity of the compression phi (nsa_phi_fwd / nsa_phi_dpre / nsa_phi_fold
behind nsa_hip_ops.phi_compress) against the float64 oracle ``phi_compress``
(pinned on the CPU: brute force, the mean-pool special case, gradcheck).

Forward output and every gradient (x, position code, W1, b1, W2, b2) meet the
strict bound (nsa_testlib.STRICT) for bf16 and float32, on overlapping
(l > d), aligned (l = d) and gapped (l < d) spans, with token counts that are
not a multiple of the 32-token tile.  The model test runs
NSAAttention(compressor='mlp') fused against 'ref' with shared weights.
"""

import pytest
import torch

from oracle import nsa_oracle as O
from nsa_testlib import assert_strict, log, randn, require_gpu

pytestmark = pytest.mark.gpu

BF, F32 = torch.bfloat16, torch.float32

# dtype, B, H, T, D, hidden, l, d
CASES = [
    (BF, 1, 4, 2048, 128, 128, 32, 16),
    (BF, 2, 2, 1000, 64, 64, 32, 16),
    (F32, 1, 3, 777, 64, 32, 16, 16),
    (BF, 2, 1, 500, 128, 64, 8, 4),
    (F32, 1, 2, 300, 128, 128, 32, 16),
    (BF, 1, 2, 401, 64, 128, 16, 20),
    (BF, 1, 2, 333, 64, 32, 5, 4),      # l D = 320: a partial 128-column group
    (F32, 2, 1, 260, 64, 64, 3, 2),     # l D = 192
]


def _rounded(t, dtype):
    """Values representable in dtype, kept in float32 (the kernels round W1 / W2)."""
    return t.to(dtype).float()


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{str(c[0])[6:]}-B{c[1]}H{c[2]}T{c[3]}D{c[4]}h{c[5]}l{c[6]}d{c[7]}")
def test_phi_matches_oracle(case):
    import nsa_hip_ops as ops
    dev = require_gpu()
    dtype, B, H, T, D, Hd, l, d = case
    log(f"phi {case}")
    x = randn((B, H, T, D), 1, dtype)
    pos = 0.3 * randn((l, D), 2, F32)
    w1 = _rounded(randn((Hd, l * D), 3, F32) * (l * D) ** -0.5, dtype)
    b1 = 0.1 * randn((Hd,), 4, F32)
    w2 = _rounded(randn((D, Hd), 5, F32) * Hd ** -0.5, dtype)
    b2 = 0.1 * randn((D,), 6, F32)
    dout = randn((B, H, O.n_cmp_tokens(T, l, d), D), 7, dtype)
    leaves = [t.to(dev).requires_grad_() for t in (x, pos, w1, b1, w2, b2)]
    out = ops.phi_compress(*leaves, l, d)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    ref_leaves = [t.double().requires_grad_() for t in (x, pos, w1, b1, w2, b2)]
    ref = O.phi_compress(*ref_leaves, l, d)
    ref.backward(dout.double())
    assert out.dtype == dtype and out.shape == ref.shape
    assert_strict(out.float().cpu(), ref, dtype, "out")
    for name, got, r in zip(["dx", "dpos", "dW1", "db1", "dW2", "db2"], leaves, ref_leaves):
        assert got.grad.dtype == got.dtype
        assert_strict(got.grad.float().cpu(), r.grad, dtype, name)


def test_phi_parameter_gradients_are_run_to_run_identical():
    """The parameter gradients are sums over every pooled token in a fixed
    order (token ranges fixed by the shape, then the ranges in order): two
    backward passes give the same bits."""
    import nsa_hip_ops as ops
    dev = require_gpu()
    B, H, T, D, Hd, l, d = 1, 4, 8192, 128, 128, 32, 16
    x = randn((B, H, T, D), 1, BF).to(dev)
    params = [(0.3 * randn((l, D), 2, F32)).to(dev), (randn((Hd, l * D), 3, F32) / 64).to(dev),
              (0.1 * randn((Hd,), 4, F32)).to(dev), (randn((D, Hd), 5, F32) / 11).to(dev),
              (0.1 * randn((D,), 6, F32)).to(dev)]
    dout = randn((B, H, O.n_cmp_tokens(T, l, d), D), 7, BF).to(dev)
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_() for t in (x, *params)]
        ops.phi_compress(*leaves, l, d).backward(dout)
        torch.cuda.synchronize()
        runs.append([t.grad.clone() for t in leaves])
    for name, a, b in zip(["dx", "dpos", "dW1", "db1", "dW2", "db2"], *runs):
        assert torch.equal(a, b), f"{name} differs between two identical backward passes"


def test_phi_model_fused_matches_ref():
    """NSAAttention(compressor='mlp'): the fused layer (phi on the HIP kernels,
    then the fused attention) against the dense 'ref' layer with the same
    weights, float32: output and every parameter gradient."""
    import nsa_model
    dev = require_gpu()
    torch.manual_seed(0)
    cfg = dict(d_model=256, n_q_heads=4, n_kv_heads=2, block_size=32, n_selected_blocks=4, window=64,
               cmp_stride=16, sel_block=64, compressor="mlp")
    ref = nsa_model.NSAAttention(**cfg, attn_impl="ref")
    for m in (ref.comp_k, ref.comp_v):   # non-trivial position codes and biases
        torch.nn.init.normal_(m.intra_pos, std=0.3)
        torch.nn.init.normal_(m.fc1.bias, std=0.1)
    fused = nsa_model.NSAAttention(**cfg, attn_impl="fused")
    fused.load_state_dict(ref.state_dict())
    ref, fused = ref.to(dev), fused.to(dev)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 512, 256, generator=g).to(dev)
    dy = torch.randn(2, 512, 256, generator=g).to(dev)
    xr, xf = x.clone().requires_grad_(), x.clone().requires_grad_()
    yr = ref(xr)
    yr.backward(dy)
    yf = fused(xf, block_idx=ref.last_block_idx)
    yf.backward(dy)
    torch.cuda.synchronize()
    err = float((yf - yr).abs().max())
    log(f"  y max_abs {err:.3e}")
    assert err <= 1e-4 * max(1.0, float(yr.abs().max()))
    assert float((xf.grad - xr.grad).abs().max()) <= 2e-3
    for (n, pr), (_, pf) in zip(sorted(ref.named_parameters()), sorted(fused.named_parameters())):
        e = float((pf.grad - pr.grad).abs().max())
        assert e <= 2e-3 * max(1.0, float(pr.grad.abs().max())), f"d{n}: {e:.3e}"
    assert any("comp_k.fc1" in n for n, _ in ref.named_parameters())
