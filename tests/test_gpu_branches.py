"""GPU parity of the three branch kernels against the float64 CPU oracle.

Selection (nsa_sel_fwd / nsa_sel_dq / nsa_sel_dkdv), window and compression
(nsa_range_fwd / nsa_range_dq / nsa_range_dkdv) through their autograd
boundaries, over the reference's kernel-test matrix (test_kernel.py:25-33)
plus GQA-16 cases, in float32 and bfloat16.  Tolerances: see nsa_testlib.TOL.
"""

import pytest
import torch

from oracle import nsa_oracle as O
from nsa_testlib import (G16_CONFIGS, REF_CONFIGS, assert_close, cfg_id, log, make_block_idx, randn,
                         require_gpu, to64, window_for)

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16]
# groups of G <= 10 heads: several selection entries per row tile (floor(32 / G)),
# with partly filled tiles (G = 5, 7, 10), two 64-key passes and ragged passes;
# the range branches number the rows (t, g) of a group t G + g (flat rows)
GP_CONFIGS = [dict(B=1, Hq=12, Hkv=2, D=64, T=512, block_size=64, S=8),
              dict(B=2, Hq=16, Hkv=2, D=32, T=640, block_size=128, S=3),
              dict(B=1, Hq=10, Hkv=1, D=128, T=384, block_size=48, S=4),
              dict(B=1, Hq=5, Hkv=1, D=64, T=333, block_size=32, S=5),
              dict(B=1, Hq=14, Hkv=2, D=64, T=400, block_size=32, S=6)]
CONFIGS = REF_CONFIGS + G16_CONFIGS + GP_CONFIGS


def _inputs(c, dtype, seed=0):
    B, Hq, Hkv, D, T = c["B"], c["Hq"], c["Hkv"], c["D"], c["T"]
    q = randn((B, Hq, T, D), seed + 1, dtype)
    k = randn((B, Hkv, T, D), seed + 2, dtype)
    v = randn((B, Hkv, T, D), seed + 3, dtype)
    do = randn((B, Hq, T, D), seed + 4, dtype)
    return q, k, v, do


def _grads_gpu(fn, q, k, v, do, dev):
    qg, kg, vg = (t.to(dev).requires_grad_() for t in (q, k, v))
    o = fn(qg, kg, vg)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    return o, qg.grad, kg.grad, vg.grad


def _grads_oracle(fn, q, k, v, do):
    q64, k64, v64, do64 = to64(q, k, v, do)
    for t in (q64, k64, v64):
        t.requires_grad_()
    o, lse = fn(q64, k64, v64)
    o.backward(do64)
    return o.detach(), lse.detach(), q64.grad, k64.grad, v64.grad


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("c", CONFIGS, ids=cfg_id)
def test_selection_fwd_bwd(c, dtype):
    dev = require_gpu()
    log(f"selection {cfg_id(c)} {dtype}")
    import nsa_selection_backward as nsb
    import nsa_selection_kernel as nsk
    q, k, v, do = _inputs(c, dtype)
    idx = make_block_idx(c["B"], c["Hkv"], c["T"], c["block_size"], c["S"])
    bs = c["block_size"]
    o_ref, lse_ref, dq_r, dk_r, dv_r = _grads_oracle(
        lambda a, b, v_: O.selection_attention(a, b, v_, idx, bs), q, k, v, do)
    o, lse = nsk.selection_forward_triton(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), bs, return_lse=True)
    assert_close(o, o_ref, dtype, "o")
    has = lse_ref > -1e8
    assert torch.equal((lse.cpu() > -1e8), has), "empty-row pattern of lse differs"
    assert_close(lse.cpu()[has], lse_ref[has], torch.float32 if dtype == torch.float32 else dtype, "lse")
    o2, dq, dk, dv = _grads_gpu(lambda a, b, v_: nsb.selection_attn_triton(a, b, v_, idx.to(dev), bs),
                                q, k, v, do, dev)
    o_fsa, _ = nsk.selection_forward_fsa(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), bs)
    assert torch.equal(o2.detach(), o_fsa), "autograd forward differs from the block-outer forward it runs"
    assert_close(o2, o_ref, dtype, "o (autograd)")
    assert_close(dq, dq_r, dtype, "dq")
    assert_close(dk, dk_r, dtype, "dk")
    assert_close(dv, dv_r, dtype, "dv")


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("c", CONFIGS, ids=cfg_id)
def test_window_fwd_bwd(c, dtype):
    dev = require_gpu()
    log(f"window {cfg_id(c)} {dtype}")
    import nsa_fused_kernel as nfk
    q, k, v, do = _inputs(c, dtype, seed=10)
    w = window_for(c)
    o_ref, _, dq_r, dk_r, dv_r = _grads_oracle(lambda a, b, v_: O.window_attention(a, b, v_, w), q, k, v, do)
    o, dq, dk, dv = _grads_gpu(lambda a, b, v_: nfk.window_attn_triton(a, b, v_, w), q, k, v, do, dev)
    assert_close(o, o_ref, dtype, "o")
    assert_close(dq, dq_r, dtype, "dq")
    assert_close(dk, dk_r, dtype, "dk")
    assert_close(dv, dv_r, dtype, "dv")


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("c", CONFIGS, ids=cfg_id)
def test_compression_fwd_bwd(c, dtype):
    """Aligned pooling (the reference's compression_attn_triton) and the
    overlapping l = 2d geometry, pooled keys as the differentiable inputs."""
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    bs = c["block_size"]
    for cl, cd in ((bs, bs), (bs, bs // 2)):
        log(f"compression {cfg_id(c)} {dtype} l={cl} d={cd}")
        q, k, v, do = _inputs(c, dtype, seed=20)
        n = O.n_cmp_tokens(c["T"], cl, cd)
        kp = O.pool_mean(k.double(), cl, cd).to(dtype)
        vp = O.pool_mean(v.double(), cl, cd).to(dtype)
        o_ref, _, dq_r, dk_r, dv_r = _grads_oracle(
            lambda a, b, v_: O.compression_attention(a, b, v_, cl, cd), q, kp, vp, do)
        o, dq, dk, dv = _grads_gpu(lambda a, b, v_: nfk.compression_attn_triton(a, b, v_, cl, cd),
                                   q, kp, vp, do, dev)
        assert dk.shape[2] == n
        assert_close(o, o_ref, dtype, "o")
        assert_close(dq, dq_r, dtype, "dq")
        assert_close(dk, dk_r, dtype, "dk")
        assert_close(dv, dv_r, dtype, "dv")


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
def test_pool_fwd_bwd(dtype):
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    x = randn((2, 3, 203, 64), 5, dtype)
    dy_shape = (2, 3, O.n_cmp_tokens(203, 32, 16), 64)
    dy = randn(dy_shape, 6, dtype)
    for cl, cd in ((32, 16), (16, 16), (64, 64)):
        x64 = x.double().requires_grad_()
        ref = O.pool_mean(x64, cl, cd)
        xg = x.to(dev).requires_grad_()
        out = nfk.block_mean_pool(xg, cl, cd)
        assert_close(out, ref, dtype, f"pool l={cl} d={cd}")
        g = randn(ref.shape, 7, dtype)
        ref.backward(g.double())
        out.backward(g.to(dev))
        assert_close(xg.grad, x64.grad, dtype, f"pool grad l={cl} d={cd}")
    del dy


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
def test_layout_helpers_both_paths(dtype):
    """transpose_kv and cast_f32 are exact copies: 16-byte-aligned inputs take
    the 8-element kernels, inputs one element off alignment the per-element ones;
    lengths that are not multiples of 8 / 64 exercise the tails and the zero pad."""
    dev = require_gpu()
    import nsa_hip_ops as ops
    for L_, D_ in ((203, 64), (64, 128), (7, 16)):
        n = 2 * 3 * L_ * D_
        flat = randn((n + 1,), 11, dtype).to(dev)
        for x in (flat[:n].view(2, 3, L_, D_), flat[1:].view(2, 3, L_, D_)):
            xt = ops.transpose_kv(x)
            Lp = ops.padded_len(L_)
            want = torch.zeros(2, 3, D_, Lp, dtype=dtype, device=dev)
            want[..., :L_] = x.transpose(-1, -2)
            assert xt.shape == want.shape and torch.equal(xt, want), (L_, D_, x.data_ptr() % 16)
    for n in (1003, 4096, 5):
        flat = randn((n + 1,), 12, torch.float32).to(dev)
        for x in (flat[:n], flat[1:]):
            y = ops.cast_f32(x, torch.bfloat16)
            assert torch.equal(y, x.to(torch.bfloat16)), (n, x.data_ptr() % 16)
    torch.cuda.synchronize()


def test_compression_dkdv_split_grid_long_sequence():
    """Compression dK/dV at T=32768 over 8 KV heads: a grid longer than one
    round of resident workgroups, so both the whole-chunk workgroups and the
    split chunks that end the grid run.  Reference: the same branch in plain
    float32 torch on the GPU (dense masked softmax; rows with no pooled key
    give 0), from the same bf16 inputs.  Tolerance: the bf16 bar of TOL."""
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    B, H, T, D, cl, cd = 1, 8, 32768, 64, 32, 16
    n = O.n_cmp_tokens(T, cl, cd)
    q = randn((B, H, T, D), 21, torch.bfloat16).to(dev)
    kp = randn((B, H, n, D), 22, torch.bfloat16).to(dev)
    vp = randn((B, H, n, D), 23, torch.bfloat16).to(dev)
    do = randn((B, H, T, D), 24, torch.bfloat16).to(dev)
    kg, vg = kp.clone().requires_grad_(), vp.clone().requires_grad_()
    nfk.compression_attn_triton(q, kg, vg, cl, cd).backward(do)
    torch.cuda.synchronize()
    t0 = cl - 1   # first query that sees a pooled token
    qf = q[:, :, t0:].float()
    kf = kp.float().requires_grad_()
    vf = vp.float().requires_grad_()
    s_ = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * D ** -0.5
    t = torch.arange(t0, T, device=dev)[:, None]
    i = torch.arange(n, device=dev)[None, :]
    s_ = s_.masked_fill(i * cd + cl - 1 > t, float("-inf"))
    o = torch.matmul(torch.softmax(s_, dim=-1), vf)
    o.backward(do[:, :, t0:].float())
    torch.cuda.synchronize()
    assert_close(kg.grad, kf.grad, torch.bfloat16, "dk")
    assert_close(vg.grad, vf.grad, torch.bfloat16, "dv")


def test_empty_and_tiny_rows():
    """T smaller than a block, all slots -1, and S = 0."""
    dev = require_gpu()
    import nsa_selection_kernel as nsk
    for T in (1, 15, 17):
        q, k, v, _ = _inputs(dict(B=1, Hq=2, Hkv=1, D=32, T=T), torch.float32)
        idx = torch.full((1, 1, T, 4), -1, dtype=torch.int32)
        o, lse = nsk.selection_forward_triton(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), 16,
                                              return_lse=True)
        assert torch.count_nonzero(o) == 0
        assert (lse == -1e9).all()


FSA_CONFIGS = CONFIGS + [dict(B=1, Hq=8, Hkv=2, D=64, T=640, block_size=128, S=3),
                         dict(B=1, Hq=16, Hkv=1, D=128, T=300, block_size=48, S=4)]


@pytest.mark.parametrize("dtype", DTYPES, ids=["f32", "bf16"])
@pytest.mark.parametrize("c", FSA_CONFIGS, ids=cfg_id)
def test_selection_fsa_and_query_outer_paths(c, dtype):
    """Both forward paths (block-outer partials + merge, query-outer) and both
    backward paths (dQ partials + reduce, query-outer dQ) against the oracle;
    blocks of 128 keys take two 64-key passes, 48-key blocks leave a ragged pass."""
    dev = require_gpu()
    log(f"selection fsa/query-outer {cfg_id(c)} {dtype}")
    import nsa_selection_backward as nsb
    import nsa_selection_kernel as nsk
    q, k, v, do = _inputs(c, dtype, seed=40)
    idx = make_block_idx(c["B"], c["Hkv"], c["T"], c["block_size"], c["S"], seed=3)
    bs = c["block_size"]
    o_ref, lse_ref, dq_r, dk_r, dv_r = _grads_oracle(
        lambda a, b, v_: O.selection_attention(a, b, v_, idx, bs), q, k, v, do)
    qd, kd, vd, dod, idd = (t.to(dev) for t in (q, k, v, do, idx))
    has = lse_ref > -1e8
    for name, fn in (("fsa", nsk.selection_forward_fsa),
                     ("query-outer", lambda *a: nsk.selection_forward_triton(*a, return_lse=True))):
        o, lse = fn(qd, kd, vd, idd, bs)
        assert_close(o, o_ref, dtype, f"o ({name})")
        assert torch.equal(lse.cpu() > -1e8, has), f"empty-row pattern of lse differs ({name})"
        assert_close(lse.cpu()[has], lse_ref[has], torch.float32 if dtype == torch.float32 else dtype, f"lse ({name})")
    o, lse = nsk.selection_forward_fsa(qd, kd, vd, idd, bs)
    for name, fn in (("fsa", lambda: nsb.selection_backward_fsa(qd, kd, vd, idd, bs, dod, o, lse)),
                     ("query-outer", lambda: nsb.selection_backward_triton(qd, kd, vd, idd, bs, dod, o))):
        dq, dk, dv = fn()
        torch.cuda.synchronize()
        assert_close(dq, dq_r, dtype, f"dq ({name})")
        assert_close(dk, dk_r, dtype, f"dk ({name})")
        assert_close(dv, dv_r, dtype, f"dv ({name})")
