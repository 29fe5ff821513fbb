"""The branch outputs the gated layer keeps for its backward, in the NSA_F16S
form: fp16 rows, each divided by a power-of-two scale, with the float32
scales after the rows.

* Stored form: for the compression forward (stored from the MFMA layout) and
  for the window forward that finishes the rows (window and merged selection
  outputs, stored in 8-element chunks), the decoded rows equal, bit for bit,
  the float32 outputs of the same launch divided by the row's scale and
  rounded once to fp16; the scale is 1 for rows below 2^15 and otherwise the
  power of two that brings the row's largest magnitude into [2^14, 2^15).
* Range: the whole layer with values far past fp16's range (the V inputs of
  one KV head scaled by 2^18) against the float64 oracle.
"""

import pytest
import torch

from oracle import nsa_oracle as O
from nsa_testlib import assert_close, log, randn, require_gpu, to64

pytestmark = pytest.mark.gpu

GEOM = dict(cmp_block=32, cmp_stride=16, sel_block=64, n_sel=8, window=128, force_init=False, n_local=0)
BIG = 2.0 ** 18


def _decode(o16):
    """(values, scales) of an NSA_F16S buffer given its float16 row view."""
    rows = o16.numel() // o16.shape[-1]
    D = o16.shape[-1]
    flat = torch.empty(0, dtype=torch.float16, device=o16.device).set_(
        o16.untyped_storage(), o16.storage_offset(), (rows * D + 2 * rows,))
    scales = flat[rows * D:].view(torch.float32).view(o16.shape[:-1])
    return o16.float() * scales[..., None], scales


def _expected(o32):
    amax = o32.abs().amax(-1)
    _, e = torch.frexp(amax)   # amax = m 2^e, m in [0.5, 1)
    scale = torch.where(amax >= 32768.0, torch.ldexp(torch.ones_like(amax), e - 15), torch.ones_like(amax))
    return (o32 / scale[..., None]).to(torch.float16).float() * scale[..., None], scale


def _check_stored(o16, o32, what):
    got, sc = _decode(o16)
    want, sc_want = _expected(o32)
    n_big = int((sc > 1).sum())
    log(f"  {what}: {n_big} of {sc.numel()} rows scaled, largest scale {float(sc.max()):.0f}")
    assert torch.equal(sc, sc_want), f"{what}: row scales differ"
    assert torch.equal(got, want), f"{what}: stored rows are not the float32 rows rounded once to fp16"
    return n_big


def _inputs(B, Hq, Hkv, T, D, seed):
    q = randn((B, Hq, T, D), seed + 1, torch.float32)
    kv = [randn((B, Hkv, T, D), seed + 2 + i, torch.float32) for i in range(6)]
    for i in (1, 3, 5):   # vc, vs, vw: KV head 0 far past fp16's range
        kv[i][:, 0] *= BIG
    gate = randn((B, Hq, T, 3), seed + 20, torch.float32)
    do = randn((B, Hq, T, D), seed + 30, torch.float32)
    return [t.to(torch.bfloat16) for t in [q] + kv + [gate]], do.to(torch.bfloat16)


@pytest.mark.parametrize("shape", [(1, 16, 2, 1024, 128), (2, 6, 2, 768, 64)], ids=["G16-D128", "G3-D64"])
def test_kept_outputs_are_fp16_rows_with_power_of_two_scales(shape):
    dev = require_gpu()
    import nsa_hip_ops as ops
    B, Hq, Hkv, T, D = shape
    log(f"f16s stored form {shape}")
    ins, _ = _inputs(B, Hq, Hkv, T, D, seed=5)
    q, kc, vc, ks, vs, kw, vw, gate = (t.to(dev) for t in ins)
    geom = ops.NSAGeometry(**GEOM)
    k_cmp = ops.pool_fwd(kc, geom.cmp_block, geom.cmp_stride)
    v_cmp = ops.pool_fwd(vc, geom.cmp_block, geom.cmp_stride)
    o_c32, lse_c = ops.range_fwd(ops.MODE_COMPRESS, q, k_cmp, v_cmp, 0, geom.cmp_block, geom.cmp_stride, o_f32=True)
    o_c16, lse_c16 = ops.range_fwd(ops.MODE_COMPRESS, q, k_cmp, v_cmp, 0, geom.cmp_block, geom.cmp_stride,
                                   o_kept=True)
    assert o_c16.dtype == torch.float16 and torch.equal(lse_c, lse_c16)
    big = _check_stored(o_c16, o_c32, "compression")
    idx = ops.importance_topn(q, k_cmp, lse_c, geom, T)
    parts, _ = ops.sel_fwd_partials(q, ks, vs, idx, geom.sel_block)
    o_w32, lse_w, o_s32, lse_s, out32 = ops.range_fwd_finish(q, kw, vw, geom.window, parts, idx, geom.sel_block,
                                                             o_c32, gate)
    o_w16, lse_w16, o_s16, lse_s16, out16 = ops.range_fwd_finish(q, kw, vw, geom.window, parts, idx,
                                                                 geom.sel_block, o_c16, gate)
    torch.cuda.synchronize()
    assert torch.equal(lse_w, lse_w16) and torch.equal(lse_s, lse_s16)
    big += _check_stored(o_w16, o_w32, "window")
    big += _check_stored(o_s16, o_s32, "selection")
    assert big > 0, "no row reached 2^15: the scaled path was not exercised"
    # the gate blends the branches as stored
    dc, _ = _decode(o_c16)
    ds, _ = _decode(o_s16)
    dw, _ = _decode(o_w16)
    sg = torch.sigmoid(gate.float())
    blend = sg[..., 0:1] * dc + sg[..., 1:2] * ds + sg[..., 2:3] * dw
    err = ((out16.float() - blend).abs() / blend.abs().clamp_min(1.0)).max()
    assert float(err) <= 2.0 ** -7, f"gated output is not the blend of the stored branches ({float(err):.2e})"


def test_layer_with_values_past_fp16_range():
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    B, Hq, Hkv, T, D = 1, 16, 2, 1024, 64
    log(f"f16s range: V of KV head 0 scaled by 2^18, B{B} Hq{Hq} Hkv{Hkv} T{T} D{D}")
    ins, do = _inputs(B, Hq, Hkv, T, D, seed=9)
    geom = ops.NSAGeometry(**GEOM)
    cfg = O.NSAConfig(**GEOM)
    xs = [t.to(dev).requires_grad_() for t in ins]
    out, idx = nfk.nsa_attention(*xs, geom)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    ins64 = [t.requires_grad_() for t in to64(*ins)]
    ref, _ = O.nsa_fused_reference(*ins64, idx.cpu(), cfg)
    ref.backward(do.double())
    assert float(ref.detach().abs().max()) > 65504.0, "the reference output must pass fp16's range"
    assert_close(out, ref.detach(), torch.bfloat16, "out")
    for nm, x, r in zip(["q", "kc", "vc", "ks", "vs", "kw", "vw", "gate"], xs, ins64):
        assert_close(x.grad, r.grad, torch.bfloat16, f"d{nm}")
