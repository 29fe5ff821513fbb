"""The dense API-parity definitions of the drop-in modules
(selection_forward_reference, _range_attn_reference, nsa_fused_reference;
nsa_selection_kernel.py:55-92, nsa_fused_kernel.py:576-609) against the
float64 oracle, on the CPU, over the reference's kernel-test matrix plus a
trailing partial block, duplicate-free -1 padding and empty rows."""

import pytest
import torch

from oracle import nsa_oracle as O
from nsa_testlib import REF_CONFIGS, cfg_id, make_block_idx, randn, window_for


def _ins(c, seed):
    B, Hq, Hkv, D, T = c["B"], c["Hq"], c["Hkv"], c["D"], c["T"]
    q = randn((B, Hq, T, D), seed + 1, torch.float32)
    kv = [randn((B, Hkv, T, D), seed + 2 + i, torch.float32) for i in range(6)]
    gate = randn((B, Hq, T, 3), seed + 9, torch.float32)
    return q, kv, gate


@pytest.mark.parametrize("c", REF_CONFIGS, ids=cfg_id)
def test_dense_definitions_match_oracle(c):
    import nsa_fused_kernel as nfk
    import nsa_selection_kernel as nsk
    q, kv, gate = _ins(c, 0)
    bs, S, T, w = c["block_size"], c["S"], c["T"], window_for(c)
    idx = make_block_idx(c["B"], c["Hkv"], T, bs, S)
    q64, kv64, g64 = q.double(), [t.double() for t in kv], gate.double()
    o, _ = O.selection_attention(q64, kv64[2], kv64[3], idx, bs)
    torch.testing.assert_close(nsk.selection_forward_reference(q, kv[2], kv[3], idx, bs).double(), o,
                               rtol=1e-5, atol=1e-5)
    o, _ = O.window_attention(q64, kv64[4], kv64[5], w)
    torch.testing.assert_close(nfk._range_attn_reference(q, kv[4], kv[5], nfk.MODE_WINDOW, w, 0).double(), o,
                               rtol=1e-5, atol=1e-5)
    kp, vp = O.pool_mean(kv64[0], bs, bs), O.pool_mean(kv64[1], bs, bs)
    o, _ = O.compression_attention(q64, kp, vp, bs, bs)
    got = nfk._range_attn_reference(q, kp.float(), vp.float(), nfk.MODE_COMPRESS, 0, bs)
    torch.testing.assert_close(got.double(), o, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(nfk._block_mean_pool_torch(kv[0], bs).double(), kp, rtol=1e-6, atol=1e-6)
    ref, _ = O.nsa_fused_reference(q64, *kv64, g64, idx, O.NSAConfig.reference(bs, S, w))
    torch.testing.assert_close(nfk.nsa_fused_reference(q, *kv, gate, idx, bs, w).double(), ref, rtol=1e-5, atol=1e-5)


def test_selection_reference_edge_rows():
    """Trailing partial block, all-empty rows (-1) and a block listed twice."""
    import nsa_selection_kernel as nsk
    B, Hq, Hkv, T, D, bs = 1, 4, 2, 100, 16, 32
    q = randn((B, Hq, T, D), 1, torch.float32)
    k = randn((B, Hkv, T, D), 2, torch.float32)
    v = randn((B, Hkv, T, D), 3, torch.float32)
    idx = make_block_idx(B, Hkv, T, bs, 3, seed=4)
    idx[:, :, 96:, -1] = 3              # tokens 96..99 through their own (partial) block
    idx[:, 0, 10] = -1                  # a row with nothing selected: output 0
    got = nsk.selection_forward_reference(q, k, v, idx, bs).double()
    o, _ = O.selection_attention(q.double(), k.double(), v.double(), idx, bs)
    torch.testing.assert_close(got, o, rtol=1e-5, atol=1e-5)
    assert float(got[0, 0:2, 10].abs().max()) == 0.0
    # listing a block twice selects it once (a set of blocks, as the mask of the reference)
    idx2 = idx.clone()
    idx2[0, 1, 70, 1] = idx2[0, 1, 70, 0]
    o2, _ = O.selection_attention(q.double(), k.double(), v.double(), idx2, bs)
    torch.testing.assert_close(nsk.selection_forward_reference(q, k, v, idx2, bs).double(), o2, rtol=1e-5, atol=1e-5)


def test_mlp_compressor_matches_oracle():
    """nsa_model.MLPCompressor on unfolded spans is the oracle's phi (the
    torch definition the fused path's HIP phi is checked against)."""
    import nsa_model
    torch.manual_seed(0)
    l, d, D = 8, 4, 16
    m = nsa_model.MLPCompressor(l, D, hidden=12).double()
    torch.nn.init.normal_(m.intra_pos, std=0.3)
    x = torch.randn(2, 3, 45, D, dtype=torch.float64)
    n = (45 - l) // d + 1
    spans = x[:, :, :(n - 1) * d + l].unfold(2, l, d).transpose(-1, -2)
    got = m(spans)
    ref = O.phi_compress(x, m.intra_pos, m.fc1.weight, m.fc1.bias, m.fc2.weight, m.fc2.bias, l, d)
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


def test_nsa_attention_mlp_compressor_ref_runs_on_cpu():
    import nsa_model
    torch.manual_seed(0)
    m = nsa_model.NSAAttention(64, 4, 2, block_size=16, n_selected_blocks=2, window=16, cmp_stride=8,
                               sel_block=32, compressor="mlp")
    x = torch.randn(2, 96, 64, requires_grad=True)
    m(x).sum().backward()
    assert m.comp_k.fc1.weight.grad is not None and torch.isfinite(m.comp_k.fc1.weight.grad).all()
    assert nsa_model.branch_of("blocks.0.attn.comp_k.fc1.weight") == "compression"
