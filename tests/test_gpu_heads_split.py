"""Head split of the stacked projection (nsa_heads_split / nsa_heads_merge_grad)
against its torch definition: per segment ``y[..., cols].view(B,T,H,hd)
.transpose(1,2)`` (nsa_model.py:192-194), plus the segment's bias, rotated
by the half-split rotary with the model's tables, in float64 on the same
inputs.  One rounding per output: bf16 within 2^-8 |ref| + 1e-5 elementwise,
float32 within 1e-5.  Gradients: the transpose, from the same cotangents."""

import pytest
import torch

pytestmark = pytest.mark.gpu

# (B, T, segments (heads, head_dim, rotate), bias segment)
CASES = [
    # the c4 NSA layer: q, kc, vc, ks, vs, kw, vw, gate
    (2, 256, [(12, 64, 1), (2, 64, 1), (2, 64, 0), (2, 64, 1), (2, 64, 0), (2, 64, 1), (2, 64, 0), (12, 3, 0)], 7),
    # c3-like head dim, no rotation, no bias
    (1, 130, [(8, 128, 0), (2, 128, 0), (2, 128, 0)], None),
    # scalar paths: head dims off the 8 / 16 channel vectors, odd columns
    (3, 37, [(2, 6, 1), (3, 5, 0), (1, 6, 1), (2, 3, 0)], 1),
    # rotated head dim a multiple of 8 but not of 16: pairs one channel a lane
    (2, 41, [(3, 24, 1), (1, 24, 1), (1, 24, 0)], None),
    # one segment
    (2, 19, [(4, 32, 1)], 0),
    # the c4 layer with the row padded to a multiple of 8 (1572 -> 1576), as the model stacks it
    (2, 64, [(12, 64, 1), (2, 64, 1), (2, 64, 0), (2, 64, 1), (2, 64, 0), (2, 64, 1), (2, 64, 0), (12, 3, 0), 4], 7),
]


def _tables(T, hd, dtype):
    import nsa_model
    return nsa_model.Rotary(hd).tables(T, "cuda", dtype)


def _reference(y, segs, cos, sin, bias, bias_seg):
    """float64 outputs of the split (the definition above)."""
    B, T, W = y.shape
    outs, col = [], 0
    y = y.double()
    for k, (H, hd, rot) in enumerate(segs):
        o = y[..., col:col + H * hd].reshape(B, T, H, hd).transpose(1, 2)
        if bias is not None and k == bias_seg:
            o = o + bias.double().view(H, hd)[None, :, None, :]
        if rot:
            h = hd // 2
            c, s = cos.double()[None, None], sin.double()[None, None]
            a, b = o[..., :h], o[..., h:]
            o = torch.cat([a * c - b * s, b * c + a * s], dim=-1)
        outs.append(o)
        col += H * hd
    return outs


def _check(got, ref, dtype):
    ref = ref.to(torch.float64)
    err = (got.double() - ref).abs()
    if dtype == torch.bfloat16:
        bound = ref.abs() * 2.0 ** -8 + 1e-5
    else:
        bound = ref.abs() * 1e-5 + 1e-5
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_heads_split_matches_definition(case, dtype):
    import nsa_hip_ops as ops
    B, T, segs, bias_seg = CASES[case]
    pad = segs[-1] if isinstance(segs[-1], int) else 0
    segs = segs[:-1] if pad else segs
    torch.manual_seed(case)
    W = sum(h * d for h, d, _ in segs) + pad
    y = torch.randn(B, T, W, device="cuda").to(dtype).requires_grad_()
    bias = None
    if bias_seg is not None:
        H, hd, _ = segs[bias_seg]
        bias = torch.randn(H * hd, device="cuda", requires_grad=True)
    rot_hd = [d for _, d, r in segs if r]
    cos, sin = _tables(T, rot_hd[0], dtype) if rot_hd else (None, None)
    print(f"[heads_split] case {case} {dtype} B{B} T{T} W{W}", flush=True)
    outs = ops.split_heads(y, segs, cos, sin, bias=bias, bias_seg=bias_seg)
    refs = _reference(y.detach(), segs, cos, sin, None if bias is None else bias.detach(), bias_seg)
    assert len(outs) == len(segs)
    for o, r in zip(outs, refs):
        assert o.shape == r.shape and o.dtype == dtype and o.is_contiguous()
        _check(o, r, dtype)

    # gradients, one output left without a gradient (a zero block of dy)
    cots = [torch.randn_like(o) for o in outs]
    skip = next((i for i in reversed(range(len(outs))) if i != bias_seg), None) if len(outs) > 1 else None
    loss = sum((o.float() * c.float()).sum() for i, (o, c) in enumerate(zip(outs, cots)) if i != skip)
    grads = torch.autograd.grad(loss, [y] + ([bias] if bias is not None else []))
    y64 = y.detach().double().requires_grad_()
    b64 = None if bias is None else bias.detach().double().requires_grad_()
    refs = _reference(y64, segs, cos, sin, b64, bias_seg)
    loss64 = sum((r * c.double()).sum() for i, (r, c) in enumerate(zip(refs, cots)) if i != skip)
    g64 = torch.autograd.grad(loss64, [y64] + ([b64] if b64 is not None else []))
    _check(grads[0], g64[0], dtype)
    if pad:
        assert bool((grads[0][..., W - pad:] == 0).all()), "padding columns get a zero gradient"
    if bias is not None:
        torch.testing.assert_close(grads[1].double(), g64[1], rtol=1e-4, atol=1e-4)


def test_heads_split_empty_sequence():
    import nsa_hip_ops as ops
    y = torch.zeros(2, 0, 96, device="cuda", dtype=torch.bfloat16)
    q, k = ops.split_heads(y, [(2, 32, 0), (1, 32, 0)])
    assert q.shape == (2, 2, 0, 32) and k.shape == (2, 1, 0, 32)


def test_heads_split_rejects_a_table_wider_than_the_row():
    import _nsa_lib as L
    import nsa_hip_ops as ops
    y = torch.zeros(1, 4, 96, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        ops.split_heads(y, [(2, 32, 0), (1, 40, 0)])
    # the library's own check, past the Python one
    heads, dims, rots, ptrs = ops._seg_table([(2, 64, 0)], [torch.empty(1, 2, 4, 64, device="cuda",
                                                                         dtype=torch.bfloat16)])
    rc = L.load().nsa_heads_split(L.ptr(y), ops._addr(ptrs), None, ops._addr(heads), ops._addr(dims),
                                  ops._addr(rots), 1, None, None, 1, 4, 96, L.dtype_code(y), L.stream_of(y))
    assert rc == L.NSA_ERR_SHAPE


@pytest.mark.parametrize("rope", [False, True], ids=["norope", "rope"])
def test_split_fused_matches_the_modules(rope):
    """The fused layer's inputs (NSAAttention._split_fused: one GEMM over the
    eight weights stacked and zero-padded, then the head split with RoPE and
    the gate bias) against each module applied on its own, split into heads
    and rotated in float64; gradients of x and of every parameter (the gate
    bias included) from the same cotangents, float32 on the GPU."""
    import nsa_model
    torch.manual_seed(0)
    Hq, Hkv, dh = 6, 2, 16
    att = nsa_model.NSAAttention(Hq * dh, Hq, Hkv, block_size=16, n_selected_blocks=2, window=32,
                                 attn_impl="fused", rope=nsa_model.Rotary(dh) if rope else None).cuda()
    with torch.no_grad():
        att.gate.bias.normal_()
    B, T = 2, 40
    x = torch.randn(B, T, Hq * dh, device="cuda", requires_grad=True)
    outs = att._split_fused(x)
    mods = (att.q_proj, att.k_cmp, att.v_cmp, att.k_slc, att.v_slc, att.k_win, att.v_win, att.gate)
    heads = (Hq, Hkv, Hkv, Hkv, Hkv, Hkv, Hkv, Hq)
    rot = (True, True, False, True, False, True, False, False)
    x64 = x.detach().double().requires_grad_()
    params64 = {n: p.detach().double().requires_grad_() for n, p in att.named_parameters()}
    cos, sin = (nsa_model.Rotary(dh).tables(T, "cpu", torch.float64) if rope else (None, None))
    refs = []
    for m, H, r in zip(mods, heads, rot):
        name = [n for n, mm in att.named_modules() if mm is m][0]
        w, b = params64[name + ".weight"], params64.get(name + ".bias")
        y = torch.nn.functional.linear(x64.cpu(), w.cpu(), None if b is None else b.cpu())
        hd = y.shape[-1] // H
        y = y.view(B, T, H, hd).transpose(1, 2)
        if r and rope:
            h2 = hd // 2
            a, c = y[..., :h2], y[..., h2:]
            y = torch.cat([a * cos - c * sin, c * cos + a * sin], dim=-1)
        refs.append(y)
    assert len(outs) == len(refs)
    for o, r in zip(outs, refs):
        assert o.shape == r.shape
        torch.testing.assert_close(o.detach().double().cpu(), r.detach(), rtol=1e-5, atol=1e-5)
    cot = [torch.randn(r.shape, dtype=torch.float64) for r in refs]
    sum((o * c.to(o.device, o.dtype)).sum() for o, c in zip(outs, cot)).backward()
    sum((r * c).sum() for r, c in zip(refs, cot)).backward()
    torch.testing.assert_close(x.grad.double().cpu(), x64.grad.cpu(), rtol=1e-5, atol=1e-5)
    for n, p in att.named_parameters():
        if n in params64 and params64[n].grad is not None:
            assert p.grad is not None, f"{n}: no gradient"
            torch.testing.assert_close(p.grad.double().cpu(), params64[n].grad.cpu(), rtol=1e-4, atol=1e-4)
