"""GPU parity of NSAAttention(attn_impl='fused') -- the HIP kernels behind the
reference's model-level flag (nsa_model.py:147-151, 306-370).

* Against the reference's golden vectors (tests/golden/nsa_model_golden.npz)
  with the reference's own block choice injected: output and every gradient
  in float32 within 1e-4 (north-star fp32 bar), relative to the largest value.
* Against attn_impl='ref' on the GPU with the same weights, mirroring the
  reference's gates (test_integration.py:24-30): the block choice is
  identical (fp32), one backward gives every parameter gradient within
  2e-3 (fp32) / 8e-2 (bf16 autocast) absolute, and the loss of 8 AdamW steps
  tracks within 5e-4 / 5e-2.
"""

import copy
import json
import os
import sys

import numpy as np
import pytest
import torch

from nsa_testlib import assert_close, log, require_gpu

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
CFG = dict(d_model=128, n_q_heads=4, n_kv_heads=2, block_size=16, n_selected_blocks=4, window=32)
B, T, STEPS = 4, 128, 8
LOSS_TOL = {torch.float32: 5e-4, torch.bfloat16: 5e-2}
GRAD_TOL = {torch.float32: 2e-3, torch.bfloat16: 8e-2}


@pytest.mark.parametrize("case", [0, 1])
def test_fused_layer_matches_reference_golden(case):
    dev = require_gpu()
    import nsa_model
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import model_params as mp
    z = np.load(os.path.join(HERE, "golden", "nsa_model_golden.npz"))
    c = json.loads(bytes(z["meta"]).decode())[case]
    name, cfg = c["name"], c["cfg"]
    log(f"model golden {name}")
    m = nsa_model.NSAAttention(**cfg, attn_impl="fused")
    mp.init_params(m, seed=1)
    m = m.to(dev)
    x, dy = mp.inputs(cfg, c["B"], c["T"], seed=2, dtype=torch.float32)
    x = x.to(dev).requires_grad_()
    y = m(x, block_idx=torch.from_numpy(z[f"{name}/topk"]).to(dev))
    y.backward(dy.to(dev))
    torch.cuda.synchronize()

    def close(got, ref, what):
        ref = torch.from_numpy(ref).double()
        err = float((got.detach().double().cpu() - ref).abs().max())
        assert err <= 1e-4 * max(1.0, float(ref.abs().max())), f"{what}: {err:.3e}"

    close(y, z[f"{name}/y"], "y")
    close(x.grad, z[f"{name}/dx"], "dx")
    for pname, p in sorted(m.named_parameters()):
        close(p.grad, z[f"{name}/grad/{pname}"], f"d{pname}")


def _snapshot():
    import nsa_model
    torch.manual_seed(0)
    return copy.deepcopy(nsa_model.NSAAttention(**CFG, attn_impl="ref").state_dict())


def _build(impl, snap, dev):
    import nsa_model
    m = nsa_model.NSAAttention(**CFG, attn_impl=impl)
    m.load_state_dict(snap)
    return m.to(dev)


def _batches(dev, n):
    g = torch.Generator().manual_seed(1)
    return [(torch.randn(B, T, CFG["d_model"], generator=g).to(dev),
             torch.randn(B, T, CFG["d_model"], generator=g).to(dev)) for _ in range(n)]


def _loss(m, x, y, dtype):
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype == torch.bfloat16):
        out = m(x)
    return ((out.float() - y) ** 2).mean()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_fused_vs_ref_grad_parity(dtype):
    dev = require_gpu()
    log(f"model grad parity {dtype}")
    snap = _snapshot()
    x, y = _batches(dev, 1)[0]
    grads, idx = {}, {}
    for impl in ("ref", "fused"):
        m = _build(impl, snap, dev)
        loss = _loss(m, x, y, dtype)
        loss.backward()
        grads[impl] = {n: p.grad.detach().float().clone() for n, p in m.named_parameters()}
        idx[impl] = m.last_block_idx.detach().cpu()
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert torch.equal(idx["ref"], idx["fused"].long().to(idx["ref"].dtype))
    worst = max(float((grads["ref"][n] - grads["fused"][n]).abs().max()) for n in grads["ref"])
    log(f"  worst |dgrad| {worst:.3e} over {len(grads['ref'])} params")
    assert worst <= GRAD_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_fused_vs_ref_loss_parity(dtype):
    dev = require_gpu()
    log(f"model loss parity {dtype}")
    snap = _snapshot()
    batches = _batches(dev, STEPS)
    losses = {}
    for impl in ("ref", "fused"):
        m = _build(impl, snap, dev)
        opt = torch.optim.AdamW(m.parameters(), lr=1e-3)
        ls = []
        for x, y in batches:
            loss = _loss(m, x, y, dtype)
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            ls.append(float(loss.detach()))
        losses[impl] = ls
    d = max(abs(a - b) for a, b in zip(losses["ref"], losses["fused"]))
    log(f"  losses ref {losses['ref'][0]:.4f}->{losses['ref'][-1]:.4f}, max |delta| {d:.2e}")
    assert d <= LOSS_TOL[dtype]


# The reference's model-level gates (test_integration.py:24-30): a two-layer
# NSATransformer, 8 AdamW steps, loss parity between attn_impl='ref' and
# 'fused', and one backward's parameter gradients.  Also the Llama-style
# variant (RMSNorm, SwiGLU, RoPE) with the BASELINE geometry shape
# (overlapping compression, larger selection blocks, forced blocks).
TF_CFG = dict(vocab_size=256, d_model=128, n_layers=2, n_q_heads=4, n_kv_heads=2, max_seq_len=128, ffn_mult=2,
              block_size=16, n_selected_blocks=4, window=32)
TF_LLAMA = dict(TF_CFG, n_q_heads=8, n_kv_heads=1, block_size=16, n_selected_blocks=5, window=48, norm="rms",
                ffn="swiglu", ffn_hidden=256, pos="rope", tie_embeddings=False, cmp_stride=8, sel_block=16,
                force_init=True, n_local=2)


def _tf_snapshot(cfg):
    import nsa_model
    torch.manual_seed(0)
    return copy.deepcopy(nsa_model.NSATransformer(attn_type="nsa", attn_impl="ref", **cfg).state_dict())


def _tf_build(cfg, impl, snap, dev):
    import nsa_model
    m = nsa_model.NSATransformer(attn_type="nsa", attn_impl=impl, **cfg)
    m.load_state_dict(snap)
    return m.to(dev)


def _tf_batches(cfg, dev, n):
    g = torch.Generator().manual_seed(1)
    return [(torch.randint(0, cfg["vocab_size"], (B, T), generator=g).to(dev),
             torch.randint(0, cfg["vocab_size"], (B, T), generator=g).to(dev)) for _ in range(n)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("variant", ["reference", "llama"])
def test_transformer_fused_vs_ref(variant, dtype):
    dev = require_gpu()
    cfg = TF_CFG if variant == "reference" else TF_LLAMA
    log(f"transformer {variant} {dtype}")
    snap = _tf_snapshot(cfg)
    batches = _tf_batches(cfg, dev, STEPS)
    amp = dtype == torch.bfloat16
    # one backward: every parameter gradient
    grads = {}
    for impl in ("ref", "fused"):
        m = _tf_build(cfg, impl, snap, dev)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
            _, loss = m(*batches[0])
        loss.backward()
        grads[impl] = {n: p.grad.detach().float().clone() for n, p in m.named_parameters() if p.grad is not None}
    assert sorted(grads["ref"]) == sorted(grads["fused"])
    worst = max(float((grads["ref"][n] - grads["fused"][n]).abs().max()) for n in grads["ref"])
    log(f"  worst |dgrad| {worst:.3e} over {len(grads['ref'])} params")
    assert worst <= GRAD_TOL[dtype]
    # loss over the AdamW steps
    losses = {}
    for impl in ("ref", "fused"):
        m = _tf_build(cfg, impl, snap, dev)
        opt = torch.optim.AdamW(m.parameters(), lr=1e-3)
        ls = []
        for x, y in batches:
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
                _, loss = m(x, y)
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            ls.append(float(loss.detach()))
        losses[impl] = ls
    torch.cuda.synchronize()
    d = max(abs(a - b) for a, b in zip(losses["ref"], losses["fused"]))
    log(f"  losses ref {losses['ref'][0]:.4f}->{losses['ref'][-1]:.4f}, max |delta| {d:.2e}")
    assert d <= LOSS_TOL[dtype]


@pytest.mark.parametrize("heads", [(12, 2), (8, 8)], ids=["gqa6", "mha"])
def test_dense_arm_sdpa_matches_ref(heads):
    """The c4 dense arm (FullAttention impl='sdpa': stacked q/k/v projection,
    flash kernels with the KV heads shared by their query groups) against the
    module's materialised causal attention (impl='ref') on the same weights,
    bf16 autocast; output and every parameter gradient."""
    import nsa_model
    dev = require_gpu()
    Hq, Hkv = heads
    torch.manual_seed(0)
    rope = nsa_model.Rotary(64)
    ref = nsa_model.FullAttention(64 * Hq, Hq, Hkv, rope=rope, impl="ref").to(dev)
    sdpa = nsa_model.FullAttention(64 * Hq, Hq, Hkv, rope=rope, impl="sdpa").to(dev)
    sdpa.load_state_dict(ref.state_dict())
    x = torch.randn(2, 256, 64 * Hq, device=dev)
    outs, grads = [], []
    for m in (ref, sdpa):
        xm = x.clone().requires_grad_()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            o = m(xm)
        o.float().square().mean().backward()
        outs.append(o.float())
        grads.append([xm.grad] + [p.grad for p in m.parameters()])
    torch.cuda.synchronize()
    assert_close(outs[1], outs[0], torch.bfloat16, "out")
    for i, (a, b) in enumerate(zip(grads[1], grads[0])):
        assert_close(a.float(), b.float(), torch.bfloat16, f"grad {i}")


@pytest.mark.gpu
@pytest.mark.parametrize("rows,d_in,d_out,bias", [(8192, 768, 1576, False), (4096, 2048, 768, True),
                                                  (4080, 64, 64, False), (1000, 96, 40, True)])
def test_split_k_linear_matches_linear(rows, d_in, d_out, bias):
    """The model's GPU linear under bf16 autocast: forward bit-identical to
    F.linear, dX within bf16 rounding, and the weight (and bias) gradient
    within 1e-4 of the float64 product: the split-K sum keeps float32 (4080
    rows: the compressors' projection at c4; rows not a multiple of 16, or
    fewer than 16 x 64, take one product with a float32 output)."""
    import nsa_model
    torch.manual_seed(rows)
    x = torch.randn(2, rows // 2, d_in, device="cuda", requires_grad=True)
    lin = nsa_model.Linear(d_in, d_out, bias=bias).cuda()
    g = torch.randn(2, rows // 2, d_out, device="cuda").bfloat16()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = lin(x)
        y_ref = torch.nn.functional.linear(x, lin.weight, lin.bias)
    assert y.dtype == torch.bfloat16 and torch.equal(y, y_ref)
    y.backward(g)
    dx, dw = x.grad.clone(), lin.weight.grad.clone()
    db = lin.bias.grad.clone() if bias else None
    x.grad = None
    lin.weight.grad = None
    y_ref.backward(g)
    assert_close(dx, x.grad, torch.bfloat16, "dx")
    xb = x.detach().bfloat16().double().reshape(-1, d_in)
    g64 = g.double().reshape(-1, d_out)
    dw64 = g64.t() @ xb
    err = (dw.double() - dw64).abs().max().item()
    print(f"[split-k linear] rows {rows} {d_in}->{d_out}: dW max err {err:.3e} of {dw64.abs().max().item():.3e}")
    assert err <= 1e-4 * dw64.abs().max().item()
    if bias:
        assert (db.double() - g64.sum(0)).abs().max().item() <= 1e-4 * g64.sum(0).abs().max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("arm", ["nsa", "full"])
def test_model_is_causal(arm):
    """Tokens at and after t0 cannot change the logits before t0: a small
    c4-like decoder (G = 6, RoPE, RMSNorm, SwiGLU, l32/d16 l'64, fused NSA or
    SDPA), bf16 autocast, every token from t0 on replaced.  t0 sits inside a
    selection block, so queries before it see that block with its later keys
    masked.  The forward's reductions never mix rows, so the logits before t0
    must be bit-identical; the ones after must change."""
    import nsa_model
    torch.manual_seed(0)
    B, T, V, t0 = 2, 1024, 512, 700
    m = nsa_model.NSATransformer(
        vocab_size=V, d_model=384, n_layers=2, n_q_heads=6, n_kv_heads=1, max_seq_len=T, ffn_hidden=768,
        norm="rms", ffn="swiglu", pos="rope", tie_embeddings=False, attn_type=arm, attn_impl="fused",
        dense_impl="sdpa", block_size=32, cmp_stride=16, sel_block=64, n_selected_blocks=4, window=128).cuda()
    x = torch.randint(0, V, (B, T), device="cuda")
    x2 = x.clone()
    x2[:, t0:] = torch.randint(0, V, (B, T - t0), device="cuda")
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        a, _ = m(x)
        b, _ = m(x2)
    assert torch.equal(a[:, :t0], b[:, :t0]), \
        f"{arm}: logits before t0 moved by {(a[:, :t0].float() - b[:, :t0].float()).abs().max().item():.3e}"
    assert not torch.equal(a[:, t0:], b[:, t0:])
