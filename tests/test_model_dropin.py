"""The drop-in modules serve the reference's own scripts (CPU).

* every name that the reference's training, test and bench scripts import
  from the five hot-path modules exists here (train.py:26,
  train_rung1.py:20-21, test_integration.py:18, smoke_integration.py:22,
  bench_e2e.py:19-20, test_kernel*.py, bench_kernel*.py, bench_range_micro.py);
* NSATransformer (attn_type 'nsa' and 'full') has the reference's state_dict
  layout and num_params(), and reproduces the reference's logits, loss and
  every parameter gradient on its golden vectors (tests/golden, written from
  the reference module on the CPU), with the reference's recorded top-k block
  choice injected per layer;
* the Llama-style options (RMSNorm, SwiGLU, RoPE, BASELINE geometry) build
  and train on the 'ref' path.
"""

import functools
import json
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

IMPORTS = {
    "nsa_model": ["NSATransformer", "param_groups", "branch_of", "REQUIRED_BRANCHES", "NSAAttention",
                  "FullAttention", "make_attention", "Block", "masked_softmax", "expand_kv", "BlockCompressor"],
    "nsa_selection_kernel": ["selection_forward_reference", "selection_forward_triton", "selection_forward_fsa",
                             "USE_FSA_FWD"],
    "nsa_selection_backward": ["selection_backward_triton", "selection_backward_fsa", "SelectionAttnTriton",
                               "selection_attn_triton", "USE_FSA_BWD"],
    "nsa_fused_kernel": ["nsa_fused_forward", "nsa_fused_reference", "block_mean_pool", "window_attn_triton",
                         "compression_attn_triton", "_RangeAttn", "_range_attn_reference", "USE_QTILE",
                         "MODE_WINDOW", "MODE_COMPRESS"],
    "nsa_fsa": ["build_block_to_query_csr"],
}


@pytest.mark.parametrize("module", sorted(IMPORTS))
def test_reference_script_imports(module):
    mod = __import__(module)
    missing = [n for n in IMPORTS[module] if not hasattr(mod, n)]
    assert not missing, f"{module} lacks {missing}"


def _golden():
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import model_params as mp
    z = np.load(os.path.join(HERE, "golden", "nsa_model_golden.npz"))
    return mp, z, json.loads(bytes(z["model_meta"]).decode())


@pytest.mark.parametrize("case", [0, 1], ids=["nsa", "full"])
def test_transformer_matches_reference_golden(case):
    import nsa_model
    mp, z, meta = _golden()
    c = meta[case]
    name, cfg = c["name"], c["cfg"]
    m = nsa_model.NSATransformer(**cfg, attn_impl="ref").double()
    layout = {k: list(v.shape) for k, v in m.state_dict().items()}
    assert layout == c["state_dict"], "state_dict layout differs from the reference's"
    assert m.num_params() == c["num_params"]
    mp.init_params(m, seed=3)
    for i in range(c["n_topk"]):
        attn = m.blocks[i].attn
        attn.forward = functools.partial(attn.forward, block_idx=torch.from_numpy(z[f"{name}/topk{i}"]))
    x, y = mp.tokens(cfg, c["B"], c["T"], seed=4)
    logits, loss = m(x, y)
    loss.backward()
    ref_logits = torch.from_numpy(z[f"{name}/logits"]).double()
    assert float((logits.detach() - ref_logits).abs().max()) <= 1e-5 * max(1.0, float(ref_logits.abs().max()))
    assert abs(float(loss) - float(z[f"{name}/loss"][0])) <= 1e-6
    n = 0
    for pname, p in sorted(m.named_parameters()):
        ref = torch.from_numpy(z[f"{name}/grad/{pname}"]).double()
        err = float((p.grad - ref).abs().max())
        assert err <= 1e-5 * max(1.0, float(ref.abs().max())), f"{pname}: {err:.3e}"
        n += 1
    assert n == sum(1 for k in z.files if k.startswith(f"{name}/grad/"))


def test_param_groups_cover_required_branches():
    import nsa_model
    m = nsa_model.NSATransformer(vocab_size=32, d_model=32, n_layers=1, n_q_heads=2, n_kv_heads=1, max_seq_len=32,
                                 block_size=8, n_selected_blocks=2, window=8)
    groups = nsa_model.param_groups(m)
    for b in nsa_model.REQUIRED_BRANCHES:
        assert b in groups and groups[b]
    assert nsa_model.branch_of("blocks.0.attn.k_slc.weight") == "selection"
    assert nsa_model.branch_of("unknown") == "other"


@pytest.mark.parametrize("attn_type", ["nsa", "full"])
def test_llama_variant_trains_on_ref_path(attn_type):
    """RMSNorm + SwiGLU + RoPE + BASELINE geometry: gradients reach every
    branch and a few AdamW steps lower the loss on a repeated batch."""
    import nsa_model
    torch.manual_seed(0)
    m = nsa_model.NSATransformer(vocab_size=64, d_model=64, n_layers=2, n_q_heads=4, n_kv_heads=2, max_seq_len=160,
                                 block_size=8, n_selected_blocks=4, window=16, attn_type=attn_type, norm="rms",
                                 ffn="swiglu", ffn_hidden=96, pos="rope", tie_embeddings=False, cmp_stride=4,
                                 sel_block=16, force_init=True, n_local=2)
    assert not hasattr(m, "pos_emb")
    assert isinstance(m.blocks[0].ln1, torch.nn.RMSNorm)
    g = torch.Generator().manual_seed(1)
    x = torch.randint(0, 64, (2, 150), generator=g)
    y = torch.randint(0, 64, (2, 150), generator=g)
    opt = torch.optim.AdamW(m.parameters(), lr=3e-3)
    losses = []
    for _ in range(6):
        _, loss = m(x, y)
        opt.zero_grad()
        loss.backward()
        if not losses and attn_type == "nsa":
            for b, ps in nsa_model.param_groups(m).items():
                if b in nsa_model.REQUIRED_BRANCHES:
                    assert any(p.grad is not None and float(p.grad.abs().sum()) > 0 for _, p in ps), b
        opt.step()
        losses.append(float(loss))
    assert losses[-1] < losses[0]


def test_rotary_is_a_rotation():
    """RoPE keeps norms and makes q.k depend on the position difference only."""
    import nsa_model
    r = nsa_model.Rotary(16)
    x = torch.randn(1, 1, 12, 16, dtype=torch.float64)
    y = r(x.float()).double()
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5, atol=1e-5)
    q = torch.randn(16, dtype=torch.float64)
    k = torch.randn(16, dtype=torch.float64)
    qs = r(q.float().expand(1, 1, 12, 16).contiguous())[0, 0].double()
    ks = r(k.float().expand(1, 1, 12, 16).contiguous())[0, 0].double()
    d1 = float(qs[5] @ ks[2])
    d2 = float(qs[9] @ ks[6])
    assert abs(d1 - d2) < 1e-4
