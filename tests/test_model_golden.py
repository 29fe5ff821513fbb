"""NSAAttention 'ref' path against golden vectors of the reference layer.

The fixture (tests/golden/nsa_model_golden.npz, written by
tests/golden/make_nsa_model_golden.py from the reference's
NSAAttention, nsa_model.py:130-304, in float64 on the CPU) holds the output,
input and parameter gradients and the block indices the reference's
``torch.topk`` returned.  Two things are pinned separately:

* the layer's arithmetic: with the reference's own block indices injected,
  output and every gradient agree to float32 rounding of the stored values;
* the block choice: on every row with at least S complete blocks (no masked
  fillers tie) our choice equals the reference's, index for index.  Rows with
  fewer complete blocks than S differ by design (ties to the lower block index;
  the reference's CPU topk picks other fillers), and the test asserts exactly
  which rows those are.
"""

import json
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "nsa_model_golden.npz")


def _load():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import model_params
    z = np.load(GOLDEN)
    meta = json.loads(bytes(z["meta"]).decode())
    return z, meta, model_params


def _layer(nsa_model, model_params, cfg, impl="ref", dtype=torch.float64, device="cpu"):
    m = nsa_model.NSAAttention(**cfg, attn_impl=impl).to(dtype)
    model_params.init_params(m, seed=1)
    return m.to(device)


def _close(got, ref, what, rtol=2e-6):
    got = got.detach().double().cpu()
    ref = torch.from_numpy(ref).double()
    scale = float(ref.abs().max()) or 1.0
    err = float((got - ref).abs().max())
    assert err <= rtol * scale + 1e-7, f"{what}: max abs err {err:.3e} (scale {scale:.3e})"


@pytest.mark.parametrize("case", [0, 1])
def test_ref_layer_matches_reference_with_its_block_choice(case):
    import nsa_model
    z, meta, mp = _load()
    c = meta[case]
    name, cfg, B, T = c["name"], c["cfg"], c["B"], c["T"]
    m = _layer(nsa_model, mp, cfg)
    x, dy = mp.inputs(cfg, B, T, seed=2)
    assert np.allclose([float(x.sum()), float(dy.sum())], z[f"{name}/input_sums"], rtol=0, atol=1e-9)
    x.requires_grad_()
    ref_idx = torch.from_numpy(z[f"{name}/topk"])
    y = m(x, block_idx=ref_idx)
    y.backward(dy)
    _close(y, z[f"{name}/y"], "y")
    _close(x.grad, z[f"{name}/dx"], "dx")
    for pname, p in sorted(m.named_parameters()):
        _close(p.grad, z[f"{name}/grad/{pname}"], f"d{pname}")


@pytest.mark.parametrize("case", [0, 1])
def test_block_choice_matches_reference_off_ties(case):
    import nsa_model
    z, meta, mp = _load()
    c = meta[case]
    name, cfg, B, T = c["name"], c["cfg"], c["B"], c["T"]
    m = _layer(nsa_model, mp, cfg)
    x, _ = mp.inputs(cfg, B, T, seed=2)
    with torch.no_grad():
        m(x)
    ours = m.last_block_idx.long()
    ref = torch.from_numpy(z[f"{name}/topk"]).long()
    L, S = cfg["block_size"], ref.shape[-1]
    t = torch.arange(T)
    full = (t + 1) // L >= S                      # at least S complete blocks: no tied fillers
    assert torch.equal(ours[:, :, full], ref[:, :, full])
    # rows with tied fillers: same valid blocks first, fillers differ by the tie rule
    for tt in torch.nonzero(~full).flatten().tolist():
        nv = (tt + 1) // L
        assert sorted(ours[0, 0, tt, :nv].tolist()) == sorted(ref[0, 0, tt, :nv].tolist()) == list(range(nv))
        assert ours[0, 0, tt, nv:].tolist() == list(range(nv, S))


@pytest.mark.parametrize("case", [0, 1])
def test_ref_layer_own_choice_matches_reference_off_ties(case):
    """With its own block choice the layer output equals the reference's on
    every row whose choice agrees (all rows with S complete blocks)."""
    import nsa_model
    z, meta, mp = _load()
    c = meta[case]
    name, cfg, B, T = c["name"], c["cfg"], c["B"], c["T"]
    m = _layer(nsa_model, mp, cfg)
    x, _ = mp.inputs(cfg, B, T, seed=2)
    with torch.no_grad():
        y = m(x)
    L, S = cfg["block_size"], z[f"{name}/topk"].shape[-1]
    full = ((torch.arange(T) + 1) // L >= S).numpy()
    _close(y[:, full], z[f"{name}/y"][:, full], "y (rows off ties)")
