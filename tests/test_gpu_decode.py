"""GPU parity of the decode path (nsa_decode_fwd, nsa_decode_append).

A decode step computes row t = lens[b] - 1 of the three-branch NSA for every
sequence from its caches (``oracle.decode_reference`` restates it; the CPU
pins show it equals the whole-sequence reference's row t).  Per case:

  (i)   the picked blocks equal the CPU top-n of the GPU's own importance
        scores, bit for bit, with -1 past S = min(n_sel, t // l' + 1);
  (ii)  the importance is within float tolerance of the float64 oracle's
        (on the GPU's pooled keys), and the end-to-end picks equal the
        oracle's except on near-tie rows (count logged);
  (iii) out and each branch's output / lse match the float64 oracle given the
        GPU's picks, to the strict bound (nsa_testlib.STRICT).

Cache rows at or past a sequence's length hold NaN, so any read beyond the
length would show.  Lengths cover the edges: 1 (only the window has keys),
below l (no pooled token), block ends and block interiors, and the full
capacity.  The append test checks the caches it builds token by token
against a prefill of the whole sequence, bit for bit.
"""

import pytest
import torch

from oracle import nsa_oracle as O
from nsa_testlib import assert_strict, log, randn, require_gpu

pytestmark = pytest.mark.gpu

BF, F32 = torch.bfloat16, torch.float32

# name, B, Hq, Hkv, D, dtype, (l, d, l', n, w, force_init, n_local), Tcap, lens
CASES = [
    ("g16-d128-c3heads", 16, 1, 128, BF, (32, 16, 64, 16, 512, False, 0), 4096,
     [4096, 1, 31, 32, 63, 64, 1000, 2049, 3333]),
    ("g4-d64-f32-aligned", 8, 2, 64, F32, (16, 16, 16, 4, 64, False, 0), 1000, [1000, 17, 500, 999]),
    ("g6-d64-forced", 12, 2, 64, BF, (32, 16, 64, 8, 128, True, 2), 2000, [2000, 700, 130]),
    ("g20-d32", 40, 2, 32, BF, (16, 8, 32, 4, 96, False, 0), 1500, [1500, 333]),
    ("g40-d16-f32-ls48", 40, 1, 16, F32, (32, 16, 48, 5, 100, True, 1), 900, [900, 47]),
    ("g16-d128-n32-long", 32, 2, 128, BF, (32, 16, 64, 32, 512, False, 0), 16384, [16384, 9000]),
    # 2048 and 2500 candidate blocks: the widest pick registers (32 / 64 per lane)
    ("g8-d32-cand2048", 8, 1, 32, BF, (32, 16, 32, 16, 256, False, 0), 65536, [65536, 40001]),
    ("g4-d32-cand2500-forced", 8, 2, 32, F32, (16, 8, 16, 24, 64, True, 2), 40000, [40000, 35001, 3]),
]


def _geom(p):
    import nsa_hip_ops as ops
    return ops.NSAGeometry(*p)


def _cfg(p):
    return O.NSAConfig(*p)


def _inputs(B, Hq, Hkv, D, dtype, Tcap, lens, seed):
    q = randn((B, Hq, D), seed, dtype)
    gate = randn((B, Hq, 3), seed + 1, dtype)
    caches = []
    for i in range(6):
        c = randn((B, Hkv, Tcap, D), seed + 2 + i, dtype)
        for b, n in enumerate(lens):
            c[b, :, n:] = float("nan")
        caches.append(c)
    return q, caches, gate


def _near_tie(sc, S, eps):
    if sc.shape[-1] <= S:
        return False
    top = torch.topk(sc, S + 1).values
    return bool((top[S - 1] - top[S]).abs() <= eps * top[S - 1].abs().clamp(min=1e-30))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(case):
    import nsa_hip_ops as ops
    dev = require_gpu()
    name, Hq, Hkv, D, dtype, gp, Tcap, lens = case
    B = len(lens)
    geom, cfg = _geom(gp), _cfg(gp)
    log(f"decode {name}: B{B} Hq{Hq} Hkv{Hkv} D{D} {dtype} Tcap{Tcap} lens {lens}")
    q, caches, gate = _inputs(B, Hq, Hkv, D, dtype, Tcap, lens, seed=100 * [c[0] for c in CASES].index(name))
    qd, gd = q.to(dev), gate.to(dev)
    cd = [c.to(dev) for c in caches]
    k_cmp = ops.pool_fwd(cd[0], geom.cmp_block, geom.cmp_stride)   # NaN where a span passes the length
    v_cmp = ops.pool_fwd(cd[1], geom.cmp_block, geom.cmp_stride)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
    out, idx, ex = ops.decode_fwd(qd, k_cmp, v_cmp, *cd[2:], gd, lens_d, geom, return_scores=True,
                                  return_branches=True)
    torch.cuda.synchronize()
    out, idx, scores = out.cpu(), idx.cpu(), ex["scores"].cpu()
    o_br, lse_br = ex["o_branch"].cpu(), ex["lse_branch"].cpu()
    q64, g64 = q.double(), gate.double()
    c64 = [c.double() for c in caches]
    kcmp64 = k_cmp.double().cpu()
    ls = geom.sel_block
    out_ref = torch.zeros(B, Hq, D, dtype=torch.float64)
    br_ref = {k: (torch.zeros(B, Hq, D, dtype=torch.float64), torch.zeros(B, Hq, dtype=torch.float64))
              for k in ("cmp", "slc", "win")}
    ties = differ = 0
    for b, n in enumerate(lens):
        t = n - 1
        ncand = t // ls + 1
        S = min(geom.n_sel, ncand)
        # (i) top-n of the GPU's own scores
        sc_gpu = scores[b, :, :ncand].double()[None, :, None]
        pick = O.topn_from_scores(O.selection_scores(sc_gpu, cfg, t_pos=[t]), S)[0, :, 0]
        assert torch.equal(pick, idx[b, :, :S]), f"b={b}: picks differ from the top-n of the GPU scores"
        assert (idx[b, :, S:] == -1).all()
        assert torch.isfinite(sc_gpu).all()
        # (ii) importance against the float64 oracle on the GPU's pooled keys
        nvis = O.n_cmp_tokens(n, geom.cmp_block, geom.cmp_stride)
        imp = O.importance_gathered(q64[b:b + 1, :, None], kcmp64[b:b + 1, :, :nvis], cfg, [t], ncand * ls)
        err = float((imp[0, :, 0] - sc_gpu[0, :, 0]).abs().max())
        assert err <= 2e-4 * max(1.0, float(imp.abs().max())), f"b={b}: importance max_abs {err:.3e}"
        sc_ref = O.selection_scores(imp, cfg, t_pos=[t])
        ref_pick = O.topn_from_scores(sc_ref, S)[0, :, 0]
        for h in range(Hkv):
            if not torch.equal(torch.sort(ref_pick[h]).values, torch.sort(idx[b, h, :S].long()).values):
                differ += 1
                tie = _near_tie(sc_ref[0, h, 0], S, 1e-4)
                ties += int(tie)
                assert tie, f"b={b} h={h}: picks differ from the oracle's outside a near tie"
        # (iii) outputs given the GPU's picks
        sl = slice(b, b + 1)
        o, br = O.nsa_rows_gathered(q64[sl, :, None], *[c[sl, :, :n] for c in c64], g64[sl, :, None],
                                    idx[sl, :, None, :S], cfg, [t], n)
        out_ref[b] = o[0, :, 0]
        for k in br_ref:
            br_ref[k][0][b] = br[k][0][0, :, 0]
            br_ref[k][1][b] = br[k][1][0, :, 0]
    log(f"  picks differing from the oracle: {differ} (all near ties: {ties})")
    assert_strict(out, out_ref, dtype, "out")
    for c, k in enumerate(("cmp", "slc", "win")):
        assert_strict(o_br[c], br_ref[k][0], F32 if dtype == F32 else dtype, f"o[{k}]")
        ref_l = br_ref[k][1]
        err = float((lse_br[c].double() - ref_l).abs().max())
        log(f"  lse[{k}] max_abs {err:.3e}")
        assert err <= 1e-3 * max(1.0, float(ref_l.abs().max()))


def test_decode_is_the_prefill_row():
    """Decode from caches holding a prefill's inputs equals that prefill's
    row t (GPU fused forward, its own top-n) -- picks except near ties, and
    outputs to the bf16 bound."""
    import nsa_hip_ops as ops
    dev = require_gpu()
    B, Hq, Hkv, T, D = 1, 32, 2, 2048, 128
    gp = (32, 16, 64, 8, 256, True, 2)
    geom = _geom(gp)
    x = [randn((B, Hq, T, D), 500, BF)] + [randn((B, Hkv, T, D), 501 + i, BF) for i in range(6)]
    gate = randn((B, Hq, T, 3), 510, BF)
    xd = [t.to(dev) for t in x]
    gd = gate.to(dev)
    out_p, idx_p = ops.nsa_attention(*xd, gd, geom)
    k_cmp = ops.pool_fwd(xd[1], geom.cmp_block, geom.cmp_stride)
    v_cmp = ops.pool_fwd(xd[2], geom.cmp_block, geom.cmp_stride)
    ts = [0, 5, 63, 64, 100, 511, 1000, 1024, 1500, 2047]
    for t in ts:
        lens = torch.tensor([t + 1], dtype=torch.int32, device=dev)
        o, idx = ops.decode_fwd(xd[0][:, :, t].contiguous(), k_cmp, v_cmp, *xd[3:], gd[:, :, t].contiguous(), lens,
                                geom)
        S = min(geom.n_sel, t // 64 + 1)
        same = torch.equal(torch.sort(idx[0, :, :S].long(), -1).values,
                           torch.sort(idx_p[0, :, t, :S].long(), -1).values)
        log(f"  t={t}: picks {'equal' if same else 'DIFFER'}")
        if same:
            assert_strict(o.float().cpu(), out_p[:, :, t].double().cpu(), BF, f"t={t}")


def test_decode_append_builds_the_prefill_caches():
    """Token-by-token appends reproduce the caches a prefill of the whole
    sequence gives, bit for bit: branch rows, pooled tokens (nsa_pool_fwd's
    sum order) and lengths; a full cache is left unchanged."""
    import nsa_hip_ops as ops
    from nsa_decode import NSADecodeCache
    dev = require_gpu()
    B, Hkv, D, Tcap = 2, 2, 64, 300
    geom = _geom((32, 16, 64, 4, 128, False, 0))
    full = [randn((B, Hkv, Tcap, D), 600 + i, BF).to(dev) for i in range(6)]
    start = [100, 37]
    cache = NSADecodeCache(B, Hkv, D, Tcap, geom, dtype=BF, device=dev)
    cache.prefill(*[f[:, :, :100] for f in full], lens=start)
    steps = Tcap - 37
    for s in range(steps):
        pos = [min(p + s, Tcap - 1) for p in start]   # sequence 0 fills up first; later rows are ignored
        rows = [torch.stack([f[b, :, pos[b]] for b in range(B)]) for f in full]
        cache.append(*rows)
    torch.cuda.synchronize()
    assert cache.lens.cpu().tolist() == [Tcap, Tcap]
    for got, ref in zip(cache.caches(), full):
        assert torch.equal(got, ref)
    n = ops.n_cmp_tokens(Tcap, geom.cmp_block, geom.cmp_stride)
    assert torch.equal(cache.k_cmp[:, :, :n], ops.pool_fwd(full[0], geom.cmp_block, geom.cmp_stride))
    assert torch.equal(cache.v_cmp[:, :, :n], ops.pool_fwd(full[1], geom.cmp_block, geom.cmp_stride))
    # a full cache: nothing written, lengths kept
    before = [c.clone() for c in cache.caches()]
    cache.append(*[torch.zeros(B, Hkv, D, device=dev, dtype=BF) for _ in range(6)])
    torch.cuda.synchronize()
    assert cache.lens.cpu().tolist() == [Tcap, Tcap]
    for a, b in zip(before, cache.caches()):
        assert torch.equal(a, b)
    # and attend on the appended caches equals attend on the prefilled ones
    q = randn((B, 8, D), 650, BF).to(dev)
    g = randn((B, 8, 3), 651, BF).to(dev)
    o1, i1 = cache.attend(q, g)
    ref = NSADecodeCache(B, Hkv, D, Tcap, geom, dtype=BF, device=dev)
    ref.prefill(*full)
    o2, i2 = ref.attend(q, g)
    torch.cuda.synchronize()
    assert torch.equal(i1, i2) and torch.equal(o1, o2)


def test_decode_generation_loop_matches_oracle():
    """A short generation loop (append + attend per step) through
    NSADecodeCache: every step's output and picks against the oracle."""
    from nsa_decode import NSADecodeCache
    dev = require_gpu()
    B, Hq, Hkv, D, Tcap = 2, 16, 2, 64, 700
    gp = (32, 16, 64, 4, 96, True, 1)
    geom, cfg = _geom(gp), _cfg(gp)
    full = [randn((B, Hkv, Tcap, D), 700 + i, BF) for i in range(6)]
    qs = randn((B, Hq, Tcap, D), 710, BF)
    gs = randn((B, Hq, Tcap, 3), 711, BF)
    cache = NSADecodeCache(B, Hkv, D, Tcap, geom, dtype=BF, device=dev)
    P = 600
    cache.prefill(*[f[:, :, :P].to(dev) for f in full])
    f64 = [f.double() for f in full]
    for t in range(P, P + 70):
        rows = [f[:, :, t].to(dev) for f in full]
        out, idx = cache.step(qs[:, :, t].to(dev), gs[:, :, t].to(dev), rows)
        if t % 10 != 3:
            continue
        out, idx = out.cpu(), idx.cpu()
        lens = torch.full((B,), t + 1)
        o_ref, i_ref, _ = O.decode_reference(qs[:, :, t].double(), *f64, gs[:, :, t].double(), lens, cfg)
        S = min(geom.n_sel, t // 64 + 1)
        for b in range(B):
            for h in range(Hkv):
                if not torch.equal(torch.sort(idx[b, h, :S].long()).values, torch.sort(i_ref[b, h, :S].long()).values):
                    log(f"  t={t} b={b} h={h}: picks differ (bf16 pooled keys vs float64)")
        # output given the GPU's picks
        outs = []
        for b in range(B):
            sl = slice(b, b + 1)
            o, _ = O.nsa_rows_gathered(qs[sl, :, t:t + 1].double(), *[f[sl, :, :t + 1] for f in f64],
                                       gs[sl, :, t:t + 1].double(), idx[sl, :, None, :S], cfg, [t], t + 1)
            outs.append(o[0, :, 0])
        assert_strict(out, torch.stack(outs), BF, f"step t={t}")


@pytest.mark.parametrize("compressor", ["mean", "mlp"])
def test_model_decode_is_the_layer_row(compressor):
    """NSAAttention.decode_cache pools with the layer's own compressor (the
    learned weighted mean + projection, or the MLP phi): a prompt prefill then
    token-by-token appends, and each step's attend equals row t of the layer's
    fused forward over the whole sequence (head-major output before the output
    projection), float32, where the two choose the same blocks.  The same
    cache without the compressor (plain span means) gives other outputs."""
    import nsa_decode
    import nsa_hip_ops as ops
    import nsa_model
    dev = require_gpu()
    torch.manual_seed(0)
    Hq, Hkv, dh, T, P = 8, 2, 64, 640, 200   # head dim 64: the phi kernels take 64 or 128
    att = nsa_model.NSAAttention(Hq * dh, Hq, Hkv, block_size=32, n_selected_blocks=4, window=96,
                                 attn_impl="fused", cmp_stride=16, sel_block=64, compressor=compressor,
                                 rope=nsa_model.Rotary(dh)).to(dev)
    with torch.no_grad():
        for p in att.parameters():
            p.add_(0.05 * torch.randn_like(p))   # pooling weights and biases away from their init
        x = torch.randn(2, T, Hq * dh, device=dev)
        q, kc, vc, ks, vs, kw, vw, gate = att._split_fused(x)
        k_cmp, v_cmp = att._pooled(kc, vc, att._n_cmp(T))
        geom = ops.NSAGeometry(32, 16, 64, 4, 96, False, 0)
        out, idx = ops.nsa_attention(q, k_cmp.to(q.dtype).contiguous(), v_cmp.to(q.dtype).contiguous(), ks, vs, kw,
                                     vw, gate, geom, pooled=True)
        cache = att.decode_cache(2, T)
        plain = nsa_decode.NSADecodeCache(2, Hkv, dh, T, geom, q.dtype, dev)
        rows = (kc, vc, ks, vs, kw, vw)
        for c in (cache, plain):
            c.prefill(*[r[:, :, :P] for r in rows])
        checked, differs = 0, 0
        for t in range(P, T):
            for c in (cache, plain):
                c.append(*[r[:, :, t] for r in rows])
            if t % 64 != 63:   # block ends: t's own block is complete for both
                continue
            o, pick = cache.attend(q[:, :, t].contiguous(), gate[:, :, t].contiguous())
            o_plain, _ = plain.attend(q[:, :, t].contiguous(), gate[:, :, t].contiguous())
            S = min(4, t // 64 + 1)
            same = torch.equal(torch.sort(pick[:, :, :S].long(), -1).values,
                               torch.sort(idx[:, :, t, :S].long(), -1).values)
            if not same:
                log(f"  t={t}: picks differ (near tie), skipped")
                continue
            err = float((o - out[:, :, t]).abs().max())
            assert err <= 1e-4, f"t={t}: decode vs the layer's row: {err:.3e}"
            differs += int(float((o_plain - out[:, :, t]).abs().max()) > 1e-3)
            checked += 1
        log(f"  {compressor}: {checked} decode rows equal the layer's rows; the plain-mean cache differs on {differs}")
        assert checked >= 6 and differs >= checked // 2
