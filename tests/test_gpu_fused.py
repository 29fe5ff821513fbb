"""GPU parity of the gated three-branch NSA, the importance / top-n block
choice and the block -> query CSR against the CPU oracle.

* nsa_fused_forward: output and the gradients of all eight differentiable
  inputs (test_kernel_fused.py:53-70) over the reference matrix.
* nsa_attention with the BASELINE geometry (l=32, d=16, l'=64, top-16 with the
  initial and two local blocks forced, w=512) on GQA-16 shapes.
* top-n: GPU indices == oracle top-n of the GPU's own scores (bit-exact),
  GPU scores within float tolerance of the oracle's, and end-to-end indices
  equal to the oracle's on every row whose S-th / (S+1)-th oracle scores are
  not a near tie.
* CSR: bit-exact equal to the oracle's restatement of nsa_fsa.py:14-64.
* nsa_pack_heads: the packed query-side layout of the selection kernels.
"""

import pytest
import torch

from oracle import nsa_oracle as O
from nsa_testlib import (REF_CONFIGS, assert_close, assert_strict, cfg_id, log, make_block_idx, randn, require_gpu,
                         to64, window_for)

pytestmark = pytest.mark.gpu

NAMES = ["q", "kc", "vc", "ks", "vs", "kw", "vw", "gate"]


def _fused_inputs(B, Hq, Hkv, T, D, dtype, seed=0, head_scale=False):
    q = randn((B, Hq, T, D), seed + 1, torch.float32)
    kv = [randn((B, Hkv, T, D), seed + 2 + i, torch.float32) for i in range(6)]
    if head_scale:
        g = torch.Generator().manual_seed(seed + 99)
        sq = torch.rand(Hq, generator=g) * 1.5 + 0.5
        skv = torch.rand(6, Hkv, generator=g) * 1.5 + 0.5
        q = q * sq[None, :, None, None]
        kv = [x * skv[i][None, :, None, None] for i, x in enumerate(kv)]
    gate = randn((B, Hq, T, 3), seed + 20, torch.float32)
    do = randn((B, Hq, T, D), seed + 30, torch.float32)
    return [t.to(dtype) for t in [q] + kv + [gate]], do.to(dtype)


def _oracle_grads(ins, do, idx, cfg):
    ins64 = to64(*ins)
    for t in ins64:
        t.requires_grad_()
    out, _ = O.nsa_fused_reference(*ins64, idx, cfg)
    out.backward(do.double())
    return out.detach(), [t.grad for t in ins64]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("c", REF_CONFIGS, ids=cfg_id)
def test_nsa_fused_forward_matches_oracle(c, dtype):
    dev = require_gpu()
    log(f"fused {cfg_id(c)} {dtype}")
    import nsa_fused_kernel as nfk
    B, Hq, Hkv, D, T, bs, S = (c[x] for x in ("B", "Hq", "Hkv", "D", "T", "block_size", "S"))
    w = window_for(c)
    ins, do = _fused_inputs(B, Hq, Hkv, T, D, dtype)
    idx = make_block_idx(B, Hkv, T, bs, S)
    cfg = O.NSAConfig.reference(bs, S, w)
    ref, gref = _oracle_grads(ins, do, idx, cfg)
    xs = [t.to(dev).requires_grad_() for t in ins]
    out = nfk.nsa_fused_forward(*xs, idx.to(dev), bs, w)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    assert_close(out, ref, dtype, "out")
    for nm, x, gr in zip(NAMES, xs, gref):
        assert_close(x.grad, gr, dtype, f"d{nm}")
    # the reference's composition of per-branch Functions gives the same result
    xs2 = [t.to(dev).requires_grad_() for t in ins]
    out2 = nfk.nsa_fused_forward_composed(*xs2, idx.to(dev), bs, w)
    out2.backward(do.to(dev))
    assert_close(out2, ref, dtype, "out (composed)")
    for nm, x, gr in zip(NAMES, xs2, gref):
        assert_close(x.grad, gr, dtype, f"d{nm} (composed)")


BASELINE_GEOM = dict(cmp_block=32, cmp_stride=16, sel_block=64, n_sel=16, window=512,
                     force_init=True, n_local=2)

SMALL_BASELINE_SHAPES = [
    dict(B=1, Hq=16, Hkv=1, T=2048, D=128),
    dict(B=1, Hq=32, Hkv=2, T=1536, D=64),
    # the c4 model's GQA group (6 heads): group-packed selection tiles, flat range rows
    dict(B=2, Hq=12, Hkv=2, T=1024, D=64),
]

# groups of at most 8 (4) heads: the top-n packs 4 (8) queries into a tile,
# each query's heads padded to 8 (4) rows
SMALL_GROUP_SHAPES = [
    dict(B=1, Hq=8, Hkv=1, T=1024, D=64),
    dict(B=1, Hq=5, Hkv=1, T=1100, D=128),
    dict(B=2, Hq=6, Hkv=2, T=1024, D=32),
    dict(B=1, Hq=4, Hkv=4, T=2048, D=128),
    dict(B=1, Hq=7, Hkv=1, T=777, D=64),
]


def _near_tie_rows(scores, S, eps):
    srt = torch.sort(scores, dim=-1, descending=True).values
    if scores.shape[-1] <= S:
        return torch.zeros(scores.shape[:-1], dtype=torch.bool)
    gap = (srt[..., S - 1] - srt[..., S]).abs()
    return gap <= eps * srt[..., S - 1].abs().clamp(min=1e-30)


def _check_topn(B, Hq, Hkv, T, D, dtype, geom_kw, qk=None):
    dev = require_gpu()
    import nsa_hip_ops as ops
    cfg = O.NSAConfig(**geom_kw)
    geom = ops.NSAGeometry(**geom_kw)
    if qk is None:
        ins, _ = _fused_inputs(B, Hq, Hkv, T, D, dtype, seed=5, head_scale=True)
        q, kc = ins[0], ins[1]
    else:
        q, kc = qk
    k_cmp = ops.pool_fwd(kc.to(dev), geom.cmp_block, geom.cmp_stride)
    _, lse_c = ops.range_fwd(ops.MODE_COMPRESS, q.to(dev), k_cmp, k_cmp, 0, geom.cmp_block, geom.cmp_stride)
    idx, scores = ops.importance_topn(q.to(dev), k_cmp, lse_c, geom, return_scores=True)
    torch.cuda.synchronize()
    idx, scores = idx.cpu(), scores.cpu()
    # (i) same scores -> same indices, bit for bit
    S = idx.shape[-1]
    sel_from_gpu_scores = O.topn_from_scores(O.selection_scores(scores.double(), cfg), S)
    assert torch.equal(sel_from_gpu_scores, idx), "top-n of identical scores differs"
    # (ii) scores within float tolerance of the oracle's (same pooled keys)
    imp_ref = O.importance(q.double(), k_cmp.cpu().double(), cfg)
    max_abs = float((scores.double() - imp_ref).abs().max())
    assert max_abs <= 2e-4 * max(1.0, float(imp_ref.abs().max())), f"importance max_abs {max_abs:.3e}"
    # (iii) end-to-end indices equal except near-tie rows
    ref_idx = O.topn_from_scores(O.selection_scores(imp_ref, cfg), S)
    tie = _near_tie_rows(O.selection_scores(imp_ref, cfg), S, 1e-4)
    rows_equal = (torch.sort(ref_idx, -1).values == torch.sort(idx, -1).values).all(-1)
    bad = (~rows_equal) & (~tie)
    log(f"  near-tie rows {int(tie.sum())} / {tie.numel()}, mismatches outside ties {int(bad.sum())}")
    assert int(bad.sum()) == 0
    # (iv) run-to-run bit identity
    idx2 = ops.importance_topn(q.to(dev), k_cmp, lse_c, geom).cpu()
    assert torch.equal(idx2, idx)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SMALL_BASELINE_SHAPES, ids=lambda s: "T{T}-Hq{Hq}-Hkv{Hkv}-D{D}".format(**s))
def test_topn_indices_bit_exact(shape, dtype):
    log(f"topn {shape} {dtype}")
    _check_topn(*(shape[x] for x in ("B", "Hq", "Hkv", "T", "D")), dtype, BASELINE_GEOM)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SMALL_GROUP_SHAPES, ids=lambda s: "T{T}-Hq{Hq}-Hkv{Hkv}-D{D}".format(**s))
def test_topn_small_groups_bit_exact(shape, dtype):
    log(f"topn small group {shape} {dtype}")
    _check_topn(*(shape[x] for x in ("B", "Hq", "Hkv", "T", "D")), dtype, BASELINE_GEOM)


# many selection blocks per query (more than 512 and more than 1024: the
# top-n phase keeps 16 and 64 block keys per lane), more picks than a wave
# has lanes, and a group of 24 heads (two 16-head chunks per tile, the
# second one half full)
MANY_BLOCK_CASES = [
    (dict(B=1, Hq=16, Hkv=1, T=4096, D=32),
     dict(cmp_block=8, cmp_stride=4, sel_block=4, n_sel=80, window=64, force_init=True, n_local=2)),
    (dict(B=1, Hq=24, Hkv=1, T=3072, D=64),
     dict(cmp_block=4, cmp_stride=2, sel_block=2, n_sel=16, window=64, force_init=False, n_local=1)),
    # 4 heads, 1024 blocks: 4 queries a tile (8 would not fit the block sums)
    (dict(B=1, Hq=4, Hkv=1, T=4096, D=64),
     dict(cmp_block=8, cmp_stride=4, sel_block=4, n_sel=40, window=64, force_init=True, n_local=2)),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("case", MANY_BLOCK_CASES, ids=["nslc1024-S80", "nslc1536-G24", "nslc1024-G4"])
def test_topn_many_blocks(case, dtype):
    shape, geom_kw = case
    log(f"topn many blocks {shape} {geom_kw} {dtype}")
    _check_topn(*(shape[x] for x in ("B", "Hq", "Hkv", "T", "D")), dtype, geom_kw)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_topn_one_lane_holds_the_best_blocks(dtype):
    """Keys zero except the selection blocks j = 5 mod 64, which hold one
    vector the queries align with: those 16 blocks tie for the best score
    and all sit in one lane's key registers (block lane + 64 k), their
    neighbours tie next in the two adjacent lanes.  The picks must take them
    in ascending block order, popping and refilling those lanes' candidate
    lists several times."""
    B, Hq, Hkv, T, D = 1, 4, 1, 4096, 64
    geom_kw = dict(cmp_block=8, cmp_stride=4, sel_block=4, n_sel=40, window=64, force_init=True, n_local=2)
    g = torch.Generator().manual_seed(11)
    v = torch.randn(D, generator=g)
    v = 4.0 * v / v.norm()
    kc = torch.zeros(B, Hkv, T, D)
    for j in range(5, T // 4, 64):
        kc[0, 0, 4 * j:4 * j + 4] = v
    q = v.expand(B, Hq, T, D).clone()
    _check_topn(B, Hq, Hkv, T, D, dtype, geom_kw, qk=(q.to(dtype), kc.to(dtype)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_topn_reference_geometry_fillers(dtype):
    """Aligned grid, no forcing: fewer valid blocks than S is filled with the
    lowest indices not chosen (the block holding t first)."""
    dev = require_gpu()
    import nsa_hip_ops as ops
    B, Hq, Hkv, T, D, bs, S = 1, 4, 1, 256, 32, 16, 6
    geom = ops.NSAGeometry.aligned(bs, S, 40)
    cfg = O.NSAConfig.reference(bs, S, 40)
    ins, _ = _fused_inputs(B, Hq, Hkv, T, D, dtype, seed=8)
    q, kc = ins[0].to(dev), ins[1].to(dev)
    k_cmp = ops.pool_fwd(kc, bs, bs)
    _, lse_c = ops.range_fwd(ops.MODE_COMPRESS, q, k_cmp, k_cmp, 0, bs, bs)
    idx, scores = ops.importance_topn(q, k_cmp, lse_c, geom, return_scores=True)
    ref = O.topn_from_scores(O.selection_scores(scores.cpu().double(), cfg), S)
    assert torch.equal(idx.cpu(), ref)
    assert idx.cpu()[0, 0, 3].tolist() == [0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SMALL_BASELINE_SHAPES, ids=lambda s: "T{T}-Hq{Hq}-Hkv{Hkv}-D{D}".format(**s))
def test_nsa_attention_baseline_geometry(shape, dtype):
    """Full NSA (GPU block choice) vs the oracle fed the GPU's block indices."""
    dev = require_gpu()
    log(f"nsa_attention {shape} {dtype}")
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    B, Hq, Hkv, T, D = (shape[x] for x in ("B", "Hq", "Hkv", "T", "D"))
    cfg = O.NSAConfig(**BASELINE_GEOM)
    geom = ops.NSAGeometry(**BASELINE_GEOM)
    ins, do = _fused_inputs(B, Hq, Hkv, T, D, dtype, seed=3, head_scale=True)
    xs = [t.to(dev).requires_grad_() for t in ins]
    out, idx = nfk.nsa_attention(*xs, geom)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    ref, gref = _oracle_grads(ins, do, idx.cpu(), cfg)
    # the BASELINE geometry and input distribution (per-head scales): the
    # elementwise north-star bound, as at the full shapes
    assert_strict(out, ref, dtype, "out")
    for nm, x, gr in zip(NAMES, xs, gref):
        assert_strict(x.grad, gr, dtype, f"d{nm}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_nsa_attention_overlapped_backward_matches_serial(dtype):
    """The backward with the selection dK/dV on a side stream gives the
    gradients of the backward run in order on one stream (up to the order of
    the float atomics), over several steps back to back."""
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    shape = SMALL_BASELINE_SHAPES[1]
    B, Hq, Hkv, T, D = (shape[x] for x in ("B", "Hq", "Hkv", "T", "D"))
    geom = ops.NSAGeometry(**BASELINE_GEOM)
    ins, do = _fused_inputs(B, Hq, Hkv, T, D, dtype, seed=11, head_scale=True)
    do = do.to(dev)

    default = ops.OVERLAP_SEL_BWD

    def grads(overlap):
        ops.OVERLAP_SEL_BWD = overlap
        try:
            res = []
            for _ in range(3):
                xs = [t.to(dev).requires_grad_() for t in ins]
                out, _ = nfk.nsa_attention(*xs, geom)
                out.backward(do)
                res.append([x.grad.float().cpu() for x in xs])
            torch.cuda.synchronize()
            return res
        finally:
            ops.OVERLAP_SEL_BWD = default

    serial = grads(False)
    overlapped = grads(True)
    for step in range(3):
        for nm, a, b in zip(NAMES, overlapped[step], serial[0]):
            assert_close(a, b, dtype, f"step {step} d{nm}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape_i", [0, 1])
def test_nsa_attention_fused_range_dq_matches_per_branch(dtype, shape_i):
    """The compression + window dQ in one launch (nsa_range_dq_cw) gives the
    gradients of one launch per branch through the float32 dQ buffer."""
    dev = require_gpu()
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    shape = SMALL_BASELINE_SHAPES[shape_i]
    B, Hq, Hkv, T, D = (shape[x] for x in ("B", "Hq", "Hkv", "T", "D"))
    geom = ops.NSAGeometry(**BASELINE_GEOM)
    ins, do = _fused_inputs(B, Hq, Hkv, T, D, dtype, seed=12, head_scale=True)
    do = do.to(dev)
    default = ops.FUSE_RANGE_DQ

    def grads(fuse):
        ops.FUSE_RANGE_DQ = fuse
        try:
            xs = [t.to(dev).requires_grad_() for t in ins]
            out, _ = nfk.nsa_attention(*xs, geom)
            out.backward(do)
            torch.cuda.synchronize()
            return [x.grad.float().cpu() for x in xs]
        finally:
            ops.FUSE_RANGE_DQ = default

    per_branch = grads(False)
    fused = grads(True)
    for nm, a, b in zip(NAMES, fused, per_branch):
        assert_close(a, b, dtype, f"d{nm}")


def test_csr_bit_exact():
    dev = require_gpu()
    import nsa_fsa
    import nsa_hip_ops as ops
    # (T 10, block 16): no complete block, an empty count matrix; 6000
    # one-token blocks: past the counting build's LDS budget, the radix sort
    for (B, Hkv, T, bs, S, seed) in ((2, 2, 256, 16, 5, 0), (1, 4, 1024, 64, 16, 1), (1, 1, 100, 32, 4, 2),
                                     (1, 2, 10, 16, 3, 4), (1, 2, 6000, 1, 4, 3)):
        idx = make_block_idx(B, Hkv, T, bs, S, seed=seed)
        # -1 padding becomes block 2: non-causal (future) for early rows, causal later
        idx[..., -1] = torch.where(idx[..., -1] < 0, torch.full_like(idx[..., -1], 2), idx[..., -1])
        q_ref, off_ref, bh_ref = O.build_block_to_query_csr(idx, bs)
        q_g, off_g, bh_g = nsa_fsa.build_block_to_query_csr(idx.to(dev), bs)
        assert torch.equal(q_g.cpu(), q_ref)
        assert torch.equal(off_g.cpu(), off_ref)
        assert torch.equal(bh_g.cpu(), bh_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_pack_heads_layout(dtype):
    """nsa_pack_heads: [B, Hkv*G, T, D] -> [B, Hkv, T, G, D], bit-exact (a pure
    permutation), including a group wider than one 16-head chunk."""
    dev = require_gpu()
    import nsa_hip_ops as ops
    for (B, Hkv, G, T, D) in ((2, 2, 4, 37, 32), (1, 1, 20, 64, 128), (1, 4, 16, 5, 16)):
        x = randn((B, Hkv * G, T, D), 7, torch.float32).to(dtype).to(dev)
        xp = ops.pack_heads(x, Hkv)
        ref = x.view(B, Hkv, G, T, D).permute(0, 1, 3, 2, 4).contiguous()
        assert xp.shape == (B, Hkv, T, G, D)
        assert torch.equal(xp, ref)


def test_csr_trailing_partial_block():
    """T not a multiple of the block: the reference grid rejects a causal pair
    on the partial block; the extended grid (used by the dK/dV kernel) keeps it."""
    dev = require_gpu()
    import nsa_fsa
    import nsa_hip_ops as ops
    B, Hkv, T, bs, S = 1, 2, 100, 32, 4
    idx = make_block_idx(B, Hkv, T, bs, S, seed=2)
    idx[:, :, 96:, -1] = 3                      # block 3 = tokens 96..99, causal for t >= 96
    with pytest.raises(IndexError):
        O.build_block_to_query_csr(idx, bs)
    with pytest.raises(IndexError):
        nsa_fsa.build_block_to_query_csr(idx.to(dev), bs)
    n_ext = -(-T // bs)
    q_ref, off_ref, bh_ref = O.build_block_to_query_csr(idx, bs, n_ext)
    q_g, off_g, bh_g, cnt = ops.csr_device(idx.to(dev), bs)
    P = int(cnt.item())
    assert P == q_ref.numel()
    assert torch.equal(q_g[:P].cpu(), q_ref)
    assert torch.equal(off_g.cpu(), off_ref)
    assert torch.equal(bh_g[:P].cpu(), bh_ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_selection_trailing_partial_block(dtype):
    """A selected trailing partial block is attended in the forward and gets its
    dK/dV in the backward (oracle: tokens past the block grid reached through
    their own block, nsa_selection_kernel.py:141-146)."""
    dev = require_gpu()
    import nsa_selection_backward as nsb
    B, Hq, Hkv, T, D, bs, S = 1, 8, 2, 100, 64, 32, 4
    q = randn((B, Hq, T, D), 1, dtype)
    k = randn((B, Hkv, T, D), 2, dtype)
    v = randn((B, Hkv, T, D), 3, dtype)
    do = randn((B, Hq, T, D), 4, dtype)
    idx = make_block_idx(B, Hkv, T, bs, S, seed=5)
    idx[:, :, 96:, -1] = 3
    q64, k64, v64, do64 = (t.double().requires_grad_() for t in (q, k, v, do))
    o_ref, _ = O.selection_attention(q64, k64, v64, idx, bs)
    o_ref.backward(do64)
    xs = [t.to(dev).requires_grad_() for t in (q, k, v)]
    o = nsb.selection_attn_triton(*xs, idx.to(dev), bs)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    assert_close(o, o_ref, dtype, "o")
    for nm, x, r in zip("qkv", xs, (q64, k64, v64)):
        assert_close(x.grad, r.grad, dtype, f"d{nm}")
    assert float(xs[1].grad[:, :, 96:].abs().max()) > 0


def _two_runs(dev, shape, geom, seed):
    import nsa_fused_kernel as nfk
    B, Hq, Hkv, T, D = shape
    ins, do = _fused_inputs(B, Hq, Hkv, T, D, torch.bfloat16, seed=seed, head_scale=True)
    runs = []
    for _ in range(2):
        xs = [t.to(dev).requires_grad_() for t in ins]
        out, idx = nfk.nsa_attention(*xs, geom)
        out.backward(do.to(dev))
        torch.cuda.synchronize()
        runs.append((out.detach().cpu(), idx.cpu(), [x.grad.float().cpu() for x in xs]))
    return runs


@pytest.mark.parametrize("shape", [(1, 16, 1, 4096, 128), (2, 12, 2, 4096, 64)], ids=["G16", "G6"])
def test_run_to_run_gradients_are_bit_identical(shape):
    """Two identical fwd+bwd steps give bit-identical block indices, output
    and every gradient.  The compression and selection dK/dV split a key's
    queries over several workgroups (at T = 4096: two 2048-query chunks and
    their split tails; selection blocks with more than 1024 pairs); their
    partial rows are summed in a fixed order, as the reference's block-outer
    dK/dV writes each block once (nsa_selection_backward.py:207-275)."""
    dev = require_gpu()
    import nsa_hip_ops as ops
    assert ops.DETERMINISTIC_DKDV
    geom = ops.NSAGeometry(**dict(BASELINE_GEOM, force_init=False, n_local=0))
    (o1, i1, g1), (o2, i2, g2) = _two_runs(dev, shape, geom, seed=21)
    assert torch.equal(i1, i2) and torch.equal(o1, o2)
    for nm, a, b in zip(NAMES, g1, g2):
        d = float((a - b).abs().max())
        log(f"  d{nm}: run-to-run max |diff| {d:.3e}")
        assert torch.equal(a, b), f"d{nm} differs between identical runs"
        assert float(a.abs().max()) > 0, f"d{nm} is all zero"


def test_atomic_dkdv_merge_is_bounded():
    """With DETERMINISTIC_DKDV off the compression and selection dK/dV merge
    their partials with float atomics: the other gradients stay bit-identical,
    those differ at most by float32 rounding of their sums."""
    dev = require_gpu()
    import nsa_hip_ops as ops
    geom = ops.NSAGeometry(**dict(BASELINE_GEOM, force_init=False, n_local=0))
    ops.DETERMINISTIC_DKDV = False
    try:
        (o1, i1, g1), (o2, i2, g2) = _two_runs(dev, (1, 16, 1, 4096, 128), geom, seed=21)
    finally:
        ops.DETERMINISTIC_DKDV = True
    assert torch.equal(i1, i2) and torch.equal(o1, o2)
    for nm, a, b in zip(NAMES, g1, g2):
        d = float((a - b).abs().max())
        rel = d / max(float(a.abs().max()), 1e-30)
        log(f"  d{nm}: run-to-run max |diff| {d:.3e} (relative {rel:.2e})")
        if nm in ("q", "gate", "kw", "vw"):
            assert d == 0.0, f"d{nm} differs between identical runs"
        else:
            assert rel <= 1e-2, f"d{nm}: run-to-run difference {rel:.2e} of its largest value"
