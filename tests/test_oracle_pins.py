"""Pins for the CPU oracle (no GPU).

The reference ships no golden vectors for this path, so each oracle function
is pinned by something independent of its own formula: a library routine it
must reduce to (SDPA with a causal mask), brute force on tiny inputs written
as explicit per-row loops, finite differences (gradcheck), closed forms and
invariants.  The last tests plant plausible mistakes in copies of the oracle
and check that a pin catches each of them.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import nsa_oracle as O


@pytest.fixture(autouse=True)
def _float64_default():
    """Every pin runs in float64; the process default is restored afterwards
    so other test modules keep torch's float32 default."""
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _rand(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64)


def _sdpa_causal(q, k, v):
    G = q.shape[1] // k.shape[1]
    return F.scaled_dot_product_attention(q, k.repeat_interleave(G, 1),
                                          v.repeat_interleave(G, 1), is_causal=True)


# ---------------------------------------------------------------- brute force

def _brute_attention(q, k, v, visible):
    """Explicit per-(b, h, t) softmax over the key list visible(b, hkv, t)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    o = torch.zeros_like(q)
    lse = torch.full((B, Hq, T), O.LSE_EMPTY)
    for b in range(B):
        for h in range(Hq):
            kh = h // G
            for t in range(T):
                keys = visible(b, kh, t)
                if not keys:
                    continue
                s = [float(q[b, h, t] @ k[b, kh, p]) * scale for p in keys]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                lse[b, h, t] = m + math.log(z)
                for p, ei in zip(keys, e):
                    o[b, h, t] += (ei / z) * v[b, kh, p]
    return o, lse


CASES = [
    dict(B=1, Hq=4, Hkv=2, T=37, D=16, l=8, d=4, ls=8, n=3, w=7),
    dict(B=2, Hq=3, Hkv=1, T=24, D=8, l=4, d=4, ls=4, n=5, w=24),
    dict(B=1, Hq=2, Hkv=2, T=33, D=8, l=16, d=8, ls=16, n=2, w=5),
]


@pytest.mark.parametrize("c", CASES)
def test_window_matches_brute_force(c):
    q = _rand(c["B"], c["Hq"], c["T"], c["D"], seed=1)
    k = _rand(c["B"], c["Hkv"], c["T"], c["D"], seed=2)
    v = _rand(c["B"], c["Hkv"], c["T"], c["D"], seed=3)
    w = c["w"]
    o, lse = O.window_attention(q, k, v, w)
    ob, lb = _brute_attention(q, k, v, lambda b, h, t: [p for p in range(max(0, t - w + 1), t + 1)])
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, lb, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("c", CASES)
def test_compression_matches_brute_force(c):
    q = _rand(c["B"], c["Hq"], c["T"], c["D"], seed=4)
    kc = _rand(c["B"], c["Hkv"], c["T"], c["D"], seed=5)
    vc = _rand(c["B"], c["Hkv"], c["T"], c["D"], seed=6)
    l, d = c["l"], c["d"]
    kp, vp = O.pool_mean(kc, l, d), O.pool_mean(vc, l, d)
    # pooled tokens by explicit means
    n = (c["T"] - l) // d + 1
    assert kp.shape[2] == n
    for i in range(n):
        torch.testing.assert_close(kp[:, :, i], kc[:, :, i * d:i * d + l].sum(2) / l)
    o, lse = O.compression_attention(q, kp, vp, l, d)
    ob, lb = _brute_attention(q, kp, vp, lambda b, h, t: [i for i in range(n) if i * d + l - 1 <= t])
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, lb, rtol=1e-12, atol=1e-12)


def _random_block_idx(B, Hkv, T, ls, S, seed=0):
    """Causal, duplicate-free block lists with -1 padding (the reference's
    test generator, test_kernel.py:39-58, restated)."""
    g = torch.Generator().manual_seed(seed)
    n_blk = T // ls
    valid = (torch.arange(n_blk)[None, :] + 1) * ls <= (torch.arange(T)[:, None] + 1)
    score = torch.rand(B, Hkv, T, n_blk, generator=g).masked_fill(~valid, -1.0)
    kk = min(S, n_blk)
    topv, topi = score.topk(kk, dim=-1)
    sel = torch.where(topv >= 0, topi.int(), torch.full_like(topi, -1, dtype=torch.int32))
    idx = torch.full((B, Hkv, T, S), -1, dtype=torch.int32)
    idx[..., :kk] = sel
    return idx


@pytest.mark.parametrize("c", CASES)
def test_selection_matches_brute_force(c):
    B, Hkv, T, ls, S = c["B"], c["Hkv"], c["T"], c["ls"], c["n"]
    q = _rand(B, c["Hq"], T, c["D"], seed=7)
    k = _rand(B, Hkv, T, c["D"], seed=8)
    v = _rand(B, Hkv, T, c["D"], seed=9)
    idx = _random_block_idx(B, Hkv, T, ls, S, seed=3)
    # also a row whose only block is the partial block containing t
    idx[0, 0, ls + 1, :] = -1
    idx[0, 0, ls + 1, 0] = 1
    o, lse = O.selection_attention(q, k, v, idx, ls)

    def vis(b, h, t):
        keys = []
        for j in idx[b, h, t].tolist():
            if j >= 0:
                keys += [p for p in range(j * ls, min((j + 1) * ls, T)) if p <= t]
        return sorted(keys)
    ob, lb = _brute_attention(q, k, v, vis)
    torch.testing.assert_close(o, ob, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, lb, rtol=1e-12, atol=1e-12)
    assert (lse == O.LSE_EMPTY).any(), "case must contain an empty row"


# ------------------------------------------------------------- library pins

def test_window_wider_than_T_is_causal_sdpa():
    q, k, v = _rand(2, 4, 50, 16, seed=1), _rand(2, 2, 50, 16, seed=2), _rand(2, 2, 50, 16, seed=3)
    o, _ = O.window_attention(q, k, v, 50)
    torch.testing.assert_close(o, _sdpa_causal(q, k, v), rtol=1e-10, atol=1e-10)


def test_all_blocks_selected_is_causal_sdpa():
    T, ls = 64, 16
    q, k, v = _rand(1, 4, T, 16, seed=4), _rand(1, 1, T, 16, seed=5), _rand(1, 1, T, 16, seed=6)
    idx = torch.arange(T // ls, dtype=torch.int32).expand(1, 1, T, T // ls).contiguous()
    o, _ = O.selection_attention(q, k, v, idx, ls)
    torch.testing.assert_close(o, _sdpa_causal(q, k, v), rtol=1e-10, atol=1e-10)


def test_unit_pool_compression_is_causal_sdpa():
    q, k, v = _rand(1, 2, 40, 8, seed=7), _rand(1, 1, 40, 8, seed=8), _rand(1, 1, 40, 8, seed=9)
    kp, vp = O.pool_mean(k, 1, 1), O.pool_mean(v, 1, 1)
    o, _ = O.compression_attention(q, kp, vp, 1, 1)
    torch.testing.assert_close(o, _sdpa_causal(q, k, v), rtol=1e-10, atol=1e-10)


def test_aligned_pool_is_reference_block_mean():
    x = _rand(2, 3, 70, 8, seed=10)
    bs = 16
    n = 70 // bs
    ref = x[:, :, :n * bs].reshape(2, 3, n, bs, 8).mean(3)      # nsa_fused_kernel.py:549-554
    torch.testing.assert_close(O.pool_mean(x, bs, bs), ref)


# ---------------------------------------------------------------- gradients

def test_gradcheck_masked_attention():
    q = _rand(1, 2, 9, 4, seed=11).requires_grad_()
    k = _rand(1, 1, 9, 4, seed=12).requires_grad_()
    v = _rand(1, 1, 9, 4, seed=13).requires_grad_()
    keep = O.window_keep(9, 4)[None, None]
    keep = keep.clone()
    keep[..., 0, :] = False                                      # one empty row
    assert torch.autograd.gradcheck(lambda a, b, c: O.masked_attention(a, b, c, keep)[0],
                                    (q, k, v))


@pytest.mark.parametrize("which", ["win", "cmp", "slc"])
def test_analytic_backward_matches_autograd(which):
    B, Hq, Hkv, T, D = 1, 4, 2, 40, 8
    q = _rand(B, Hq, T, D, seed=20).requires_grad_()
    k = _rand(B, Hkv, T, D, seed=21)
    v = _rand(B, Hkv, T, D, seed=22)
    if which == "win":
        keep = O.window_keep(T, 7)[None, None]
    elif which == "cmp":
        k, v = O.pool_mean(k, 8, 4), O.pool_mean(v, 8, 4)
        keep = O.compress_keep(T, k.shape[2], 8, 4)[None, None]
    else:
        keep = O.select_keep(_random_block_idx(B, Hkv, T, 8, 3, seed=1), T, 8)
    k.requires_grad_()
    v.requires_grad_()
    do = _rand(B, Hq, T, D, seed=23)
    o, _ = O.masked_attention(q, k, v, keep)
    o.backward(do)
    dq, dk, dv = O.attention_backward(q.detach(), k.detach(), v.detach(), keep, do)
    torch.testing.assert_close(dq, q.grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dk, k.grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dv, v.grad, rtol=1e-10, atol=1e-10)


def test_gradcheck_full_nsa_tiny():
    cfg = O.NSAConfig(cmp_block=4, cmp_stride=2, sel_block=4, n_sel=2, window=3,
                      force_init=True, n_local=2)
    B, Hq, Hkv, T, D = 1, 2, 1, 12, 4
    ins = [_rand(B, Hq, T, D, seed=30)] + [_rand(B, Hkv, T, D, seed=31 + i) for i in range(6)] \
        + [_rand(B, Hq, T, 3, seed=40)]
    ins = [t.requires_grad_() for t in ins]
    idx = O.select_blocks(ins[0].detach(), O.pool_mean(ins[1].detach(), 4, 2), cfg)[0]

    def f(*a):
        return O.nsa_fused_reference(*a, idx, cfg)[0]
    assert torch.autograd.gradcheck(f, tuple(ins))


# ------------------------------------------------------------- importance/topn

def test_overlap_weights_identity_when_aligned():
    W = O.overlap_weights(8, 8, 16, 16, 16)
    torch.testing.assert_close(W, torch.eye(8))


def test_overlap_weights_nsa_paper_pattern():
    W = O.overlap_weights(n_cmp=31, n_slc=8, l=32, d=16, ls=64)
    for j in range(1, 7):
        col = W[:, j]
        nz = torch.nonzero(col).flatten().tolist()
        assert nz == [4 * j - 1, 4 * j, 4 * j + 1, 4 * j + 2, 4 * j + 3]
        assert col[nz].tolist() == [1.0, 2.0, 2.0, 2.0, 1.0]
    # every token fully inside the grid distributes l/d in total
    torch.testing.assert_close(W[:29].sum(1), torch.full((29,), 2.0))


def test_importance_matches_brute_force():
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=3, window=8)
    B, Hq, Hkv, T, D = 1, 4, 2, 48, 8
    q = _rand(B, Hq, T, D, seed=50)
    kc = _rand(B, Hkv, T, D, seed=51)
    kp = O.pool_mean(kc, 8, 4)
    n = kp.shape[2]
    imp = O.importance(q, kp, cfg)
    G = Hq // Hkv
    for b in range(B):
        for hk in range(Hkv):
            for t in range(T):
                vis = [i for i in range(n) if i * 4 + 8 - 1 <= t]
                pc = [0.0] * n
                for g in range(G):
                    h = hk * G + g
                    if not vis:
                        continue
                    s = [float(q[b, h, t] @ kp[b, hk, i]) / math.sqrt(D) for i in vis]
                    m = max(s)
                    z = sum(math.exp(x - m) for x in s)
                    for i, x in zip(vis, s):
                        pc[i] += math.exp(x - m) / z
                for j in range(T // 16):
                    ref = 0.0
                    for i in range(n):
                        ov = max(0, min(i * 4 + 8, (j + 1) * 16) - max(i * 4, j * 16))
                        ref += ov / 4 * pc[i]
                    assert abs(float(imp[b, hk, t, j]) - ref) < 1e-12


def _brute_topn(scores_row, S):
    order = sorted(range(len(scores_row)), key=lambda j: (-scores_row[j], j))
    return order[:S]


def test_topn_ties_go_to_lower_index():
    sc = torch.tensor([[[[1.0, 3.0, 3.0, 0.5, 3.0, O.F32_MIN, O.F32_MIN, 2.0]]]])
    assert O.topn_from_scores(sc, 5).flatten().tolist() == [1, 2, 4, 7, 0]
    assert O.topn_from_scores(sc, 8).flatten().tolist() == [1, 2, 4, 7, 0, 3, 5, 6]


def test_topn_matches_brute_force_with_mask_and_forcing():
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=8, n_sel=5, window=8,
                      force_init=True, n_local=2)
    g = torch.Generator().manual_seed(3)
    T, n_slc = 80, 10
    imp = torch.rand(1, 2, T, n_slc, generator=g).round(decimals=1)  # many exact ties
    sc = O.selection_scores(imp, cfg)
    idx = O.topn_from_scores(sc, 5)
    for h in range(2):
        for t in range(T):
            row = []
            for j in range(n_slc):
                forced = j == 0 or j in (t // 8, t // 8 - 1)
                if forced:
                    row.append(math.inf)
                elif (j + 1) * 8 - 1 <= t:
                    row.append(float(imp[0, h, t, j]))
                else:
                    row.append(O.F32_MIN)
            assert idx[0, h, t].tolist() == _brute_topn(row, 5), (h, t)


def test_topn_reference_mode_fillers():
    """Aligned grid, no forcing: rows with fewer valid blocks than S take the
    lowest non-valid indices, starting with the block that contains t."""
    cfg = O.NSAConfig.reference(16, 4, 16)
    imp = torch.rand(1, 1, 64, 4)
    idx = O.topn_from_scores(O.selection_scores(imp, cfg), 4)
    assert idx[0, 0, 5].tolist() == [0, 1, 2, 3]                 # nothing complete yet
    row = idx[0, 0, 20].tolist()                                 # block 0 complete
    assert row[0] == 0 and row[1:] == [1, 2, 3]
    row = idx[0, 0, 40].tolist()                                 # blocks 0,1 complete
    assert sorted(row[:2]) == [0, 1] and row[2:] == [2, 3]


# ---------------------------------------------------------------- CSR

def test_csr_invariants_and_counts():
    B, Hkv, T, ls, S = 2, 2, 64, 8, 4
    idx = _random_block_idx(B, Hkv, T, ls, S, seed=7)
    idx[0, 0, 3, 0] = 0          # a non-causal pair (block 0 starts at 0 <= 3: causal)
    idx[0, 0, 3, 1] = 5          # block 5 starts at 40 > 3: must be dropped
    idx[1, 1, 40, 3] = idx[1, 1, 40, 0]   # a block listed twice: two pairs
    qob, off, pbh = O.build_block_to_query_csr(idx, ls)
    n_blk = T // ls
    # brute force: walk blocks, then queries, then slots
    ref_q, ref_off, ref_bh = [], torch.zeros(B, Hkv, n_blk + 1, dtype=torch.int32), []
    for b in range(B):
        for h in range(Hkv):
            for j in range(n_blk):
                ref_off[b, h, j] = len(ref_q)
                for t in range(T):
                    for s in range(S):
                        if int(idx[b, h, t, s]) == j and j * ls <= t:
                            ref_q.append(t)
                            ref_bh.append(b * Hkv + h)
            ref_off[b, h, n_blk] = len(ref_q)
    assert qob.tolist() == ref_q
    assert pbh.tolist() == ref_bh
    assert torch.equal(off, ref_off)
    assert (off[..., 1:] >= off[..., :-1]).all()
    for b in range(B):
        for h in range(Hkv):
            for j in range(n_blk):
                seg = qob[off[b, h, j]:off[b, h, j + 1]].long()
                assert (seg[1:] >= seg[:-1]).all()                      # ascending
                assert (seg >= j * ls).all()                            # causal


def test_csr_trailing_partial_block():
    """Reference grid (T // ls): a causal pair on the partial block raises, like
    the reference's scatter_add_ into n_blk columns; the ceil grid keeps it as
    its own last block (brute force)."""
    B, Hkv, T, ls, S = 1, 1, 50, 16, 3
    idx = _random_block_idx(B, Hkv, T, ls, S, seed=3)
    idx[0, 0, 49, 2] = 3                       # tokens 48..49, causal for t = 49
    with pytest.raises(IndexError):
        O.build_block_to_query_csr(idx, ls)
    qob, off, pbh = O.build_block_to_query_csr(idx, ls, 4)
    assert off.shape == (1, 1, 5)
    assert qob[off[0, 0, 3]:off[0, 0, 4]].tolist() == [49]
    idx[0, 0, 20, 2] = 3                       # block 3 starts at 48 > 20: dropped, no error
    idx[0, 0, 49, 2] = -1
    O.build_block_to_query_csr(idx, ls)


# ------------------------------------------------------------- rows vs dense

def test_rows_path_matches_dense_path():
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=3, window=10,
                      force_init=True, n_local=2)
    B, Hq, Hkv, T, D = 1, 4, 2, 96, 8
    q = _rand(B, Hq, T, D, seed=60)
    kv = [_rand(B, Hkv, T, D, seed=61 + i) for i in range(6)]
    gate = _rand(B, Hq, T, 3, seed=70)
    out, parts = O.nsa_forward_reference(q, *kv, gate, cfg)
    rows = torch.tensor([0, 1, 7, 15, 16, 33, 64, 95])
    out_r, parts_r = O.nsa_rows(q, *kv, gate, parts["block_idx"], cfg, rows)
    torch.testing.assert_close(out_r, out[:, :, rows], rtol=1e-12, atol=1e-12)
    for key in ("cmp", "slc", "win"):
        torch.testing.assert_close(parts_r[key][1], parts[key][1][:, :, rows])
    imp_r = O.importance_rows(q, parts["k_cmp"], cfg, rows, T)
    torch.testing.assert_close(imp_r, parts["importance"][:, :, rows])
    o_s, lse_s = O.selection_rows(q[:, :, rows], kv[2], kv[3], parts["block_idx"][:, :, rows], 16, rows, T)
    torch.testing.assert_close(o_s, parts["slc"][0][:, :, rows], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse_s, parts["slc"][1][:, :, rows])


def test_rows_path_gradients_match_dense_path():
    """Gradients through the row path (row inputs as their own leaves) equal
    the dense path's with dO zero outside the rows."""
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=3, window=10)
    B, Hq, Hkv, T, D = 1, 4, 2, 80, 8
    q = _rand(B, Hq, T, D, seed=80)
    kv = [_rand(B, Hkv, T, D, seed=81 + i) for i in range(6)]
    gate = _rand(B, Hq, T, 3, seed=90)
    rows = torch.tensor([0, 9, 31, 32, 50, 79])
    dor = _rand(B, Hq, rows.numel(), D, seed=91)
    xs = [t.clone().requires_grad_() for t in [q] + kv + [gate]]
    out, parts = O.nsa_forward_reference(*xs, cfg)
    do = torch.zeros_like(out)
    do[:, :, rows] = dor
    out.backward(do)
    idx = parts["block_idx"]
    qr = q[:, :, rows].clone().requires_grad_()
    gr = gate[:, :, rows].clone().requires_grad_()
    ys = [t.clone().requires_grad_() for t in kv]
    out_r, _ = O.nsa_rows_gathered(qr, *ys, gr, idx[:, :, rows], cfg, rows, T)
    out_r.backward(dor)
    torch.testing.assert_close(qr.grad, xs[0].grad[:, :, rows], rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(gr.grad, xs[7].grad[:, :, rows], rtol=1e-10, atol=1e-12)
    for a, b in zip(ys, xs[1:7]):
        torch.testing.assert_close(a.grad, b.grad, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("cfg", [
    O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=3, window=10, force_init=True, n_local=2),
    O.NSAConfig(cmp_block=16, cmp_stride=16, sel_block=16, n_sel=2, window=24),
    O.NSAConfig(cmp_block=8, cmp_stride=8, sel_block=12, n_sel=4, window=7),
])
def test_decode_step_is_the_prefill_row(cfg):
    """A decode step at t (caches holding tokens 0..t, garbage above) equals
    row t of the whole-sequence NSA of a sequence whose length is a multiple
    of the selection block: the same block choice and the same output."""
    B, Hq, Hkv, T, D = 2, 4, 2, 96, 8
    assert T % cfg.sel_block == 0
    q = _rand(B, Hq, T, D, seed=100)
    kv = [_rand(B, Hkv, T, D, seed=101 + i) for i in range(6)]
    gate = _rand(B, Hq, T, 3, seed=110)
    out, parts = O.nsa_forward_reference(q, *kv, gate, cfg)
    idx_full = parts["block_idx"]
    for t in [0, 3, 7, 8, 15, 16, 17, 31, 40, 47, 48, 63, 95]:
        lens = torch.tensor([t + 1, max(1, t - 5)])
        caches = [x.clone() for x in kv]
        for c in caches:   # rows at or past lens[b] must not matter
            for b in range(B):
                c[b, :, int(lens[b]):] = float("nan")
        qd = torch.stack([q[0, :, t], q[1, :, int(lens[1]) - 1]])
        gd = torch.stack([gate[0, :, t], gate[1, :, int(lens[1]) - 1]])
        o_d, i_d, p_d = O.decode_reference(qd, *caches, gd, lens, cfg)
        for b in range(B):
            tb = int(lens[b]) - 1
            torch.testing.assert_close(o_d[b], out[b, :, tb], rtol=1e-12, atol=1e-12)
            S = min(cfg.n_sel, tb // cfg.sel_block + 1)
            assert torch.equal(i_d[b, :, :S], idx_full[b, :, tb, :S]), (t, b)
            assert (i_d[b, :, S:] == -1).all()
            ncand = tb // cfg.sel_block + 1
            torch.testing.assert_close(p_d[b]["importance"], parts["importance"][b, :, tb, :ncand])


def test_decode_empty_cache_is_zero():
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=3, window=10)
    q, gate = _rand(1, 2, 8, seed=1), _rand(1, 2, 3, seed=2)
    kv = [_rand(1, 1, 16, 8, seed=3 + i) for i in range(6)]
    o, idx, parts = O.decode_reference(q, *kv, gate, torch.tensor([0]), cfg)
    assert (o == 0).all() and (idx == -1).all() and parts == [None]


# ------------------------------------------------------------- compression phi

def _phi_params(l, D, Hd, seed):
    return (0.3 * _rand(l, D, seed=seed), 0.05 * _rand(Hd, l * D, seed=seed + 1), 0.1 * _rand(Hd, seed=seed + 2),
            0.2 * _rand(D, Hd, seed=seed + 3), 0.1 * _rand(D, seed=seed + 4))


def test_phi_identity_mean_is_pool_mean():
    """With the identity activation, W1 averaging each channel over the span,
    W2 = I and no position code or bias, phi is the mean pool."""
    l, d, D = 8, 4, 6
    x = _rand(2, 3, 41, D, seed=120)
    w1 = torch.zeros(D, l * D)
    for p in range(l):
        w1[:, p * D:(p + 1) * D] = torch.eye(D) / l
    out = O.phi_compress(x, torch.zeros(l, D), w1, torch.zeros(D), torch.eye(D), torch.zeros(D), l, d,
                         act="identity")
    torch.testing.assert_close(out, O.pool_mean(x, l, d), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("l,d", [(8, 4), (4, 4), (6, 3), (5, 7)])
def test_phi_matches_brute_force(l, d):
    D, Hd, T = 3, 5, 29
    x = _rand(1, 2, T, D, seed=130)
    pos, w1, b1, w2, b2 = _phi_params(l, D, Hd, 131)
    out = O.phi_compress(x, pos, w1, b1, w2, b2, l, d)
    n = (T - l) // d + 1
    assert out.shape == (1, 2, n, D)
    for h in range(2):
        for i in range(n):
            pre = [float(b1[u]) + sum(float(w1[u, p * D + c]) * (float(x[0, h, i * d + p, c]) + float(pos[p, c]))
                                      for p in range(l) for c in range(D)) for u in range(Hd)]
            hid = [z / (1.0 + math.exp(-z)) for z in pre]
            for c in range(D):
                ref = float(b2[c]) + sum(float(w2[c, u]) * hid[u] for u in range(Hd))
                assert abs(float(out[0, h, i, c]) - ref) < 1e-12


def test_phi_gradcheck():
    l, d, D, Hd = 4, 2, 3, 4
    x = _rand(1, 1, 11, D, seed=140).requires_grad_()
    ps = [t.requires_grad_() for t in _phi_params(l, D, Hd, 141)]
    assert torch.autograd.gradcheck(lambda *a: O.phi_compress(*a, l, d), (x, *ps))


def test_keys_per_row_matches_masks():
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=3, window=10)
    T = 96
    idx = _random_block_idx(1, 2, T, 16, 3, seed=9)
    kw, kc, ksel = O.keys_per_row(T, cfg, idx)
    assert kw == int(O.window_keep(T, 10).sum())
    n = O.n_cmp_tokens(T, 8, 4)
    assert kc == int(O.compress_keep(T, n, 8, 4).sum())
    assert ksel == int(O.select_keep(idx, T, 16).sum())


# ------------------------------------------------------- planted mistakes

def test_pins_catch_planted_mistakes():
    """Each mutated oracle variant must fail at least one pin above."""
    q, k, v = _rand(1, 2, 30, 8, seed=1), _rand(1, 1, 30, 8, seed=2), _rand(1, 1, 30, 8, seed=3)
    w = 6
    good = [p for p in range(30)]
    ob, _ = _brute_attention(q, k, v, lambda b, h, t: [p for p in range(max(0, t - w + 1), t + 1)])
    # window off by one (t - p <= w)
    t_ = torch.arange(30)[:, None]
    p_ = torch.arange(30)[None, :]
    bad_keep = (p_ <= t_) & (t_ - p_ <= w)
    o_bad, _ = O.masked_attention(q, k, v, bad_keep[None, None])
    assert not torch.allclose(o_bad, ob)
    # wrong GQA mapping (h % Hkv instead of h // G) on Hkv=2
    k2, v2 = _rand(1, 2, 30, 8, seed=4), _rand(1, 2, 30, 8, seed=5)
    q4 = _rand(1, 4, 30, 8, seed=6)
    o_ok, _ = O.window_attention(q4, k2, v2, 30)
    o_bad = _sdpa_causal(q4, k2[:, [0, 1, 0, 1]], v2[:, [0, 1, 0, 1]])
    assert torch.allclose(o_ok, _sdpa_causal(q4, k2, v2))
    assert not torch.allclose(o_ok, o_bad)
    # compression visibility shifted by one token (i*d + l <= t)
    kp, vp = O.pool_mean(k, 4, 4), O.pool_mean(v, 4, 4)
    n = kp.shape[2]
    bad = (torch.arange(n)[None, :] * 4 + 4 <= torch.arange(30)[:, None])
    o_bad, _ = O.masked_attention(q, kp, vp, bad[None, None])
    ob, _ = _brute_attention(q, kp, vp, lambda b, h, t: [i for i in range(n) if i * 4 + 3 <= t])
    assert not torch.allclose(o_bad, ob)
    # dropped delta term in dS
    keep = O.window_keep(30, 30)[None, None]
    do = _rand(1, 2, 30, 8, seed=7)
    dq, _, _ = O.attention_backward(q, k, v, keep, do)
    p = O.attention_probs(q, k, keep)
    dq_bad = (8 ** -0.5) * (p * (do @ v.repeat_interleave(2, 1).transpose(-1, -2))) @ k.repeat_interleave(2, 1)
    assert not torch.allclose(dq, dq_bad)
    # decode offering complete blocks only (ncand = len // ls): differs from
    # the prefill row where t sits inside a block with local forcing
    cfg = O.NSAConfig(cmp_block=8, cmp_stride=4, sel_block=16, n_sel=2, window=4, n_local=1)
    qq = _rand(1, 2, 64, 8, seed=20)
    kvs = [_rand(1, 1, 64, 8, seed=21 + i) for i in range(6)]
    gg = _rand(1, 2, 64, 3, seed=30)
    _, parts = O.nsa_forward_reference(qq, *kvs, gg, cfg)
    t = 40
    kcmp = O.pool_mean(kvs[0][:, :, :t + 1], 8, 4)
    imp = O.importance_gathered(qq[:, :, t:t + 1], kcmp, cfg, [t], t + 1)
    bad = O.topn_from_scores(O.selection_scores(imp, cfg, t_pos=[t]), min(2, imp.shape[-1]))
    assert not torch.equal(bad[0, :, 0], parts["block_idx"][0, :, t])
    # phi with the spans one token late (x[i*d+1 : i*d+l+1]) fails the brute force
    xs = _rand(1, 1, 20, 3, seed=150)
    pos, w1, b1, w2, b2 = _phi_params(4, 3, 5, 151)
    good_phi = O.phi_compress(xs, pos, w1, b1, w2, b2, 4, 2)
    bad_phi = O.phi_compress(xs[:, :, 1:], pos, w1, b1, w2, b2, 4, 2)[:, :, :good_phi.shape[2] - 1]
    assert not torch.allclose(good_phi[:, :, :bad_phi.shape[2]], bad_phi)
    # top-n tie broken toward the higher index
    sc = torch.tensor([[[[2.0, 2.0, 1.0]]]])
    assert O.topn_from_scores(sc, 1).item() == 0
    assert torch.sort(sc, descending=True).indices[..., 0].item() in (0, 1)
    del good
