"""NSA fused forward + backward throughput on one MI355X.

A step is one full NSA attention layer call, forward and backward, over one
batch of synthetic inputs resident in HBM: compression pooling, compression
attention, block importance + top-n on the GPU, selection and sliding-window
attention, gate blend, then the backward of all of it.  The default workload
is BASELINE config 3 as stated there: B1 T32768 Hq64 Hkv4 D128, l=32 d=16
l'=64, plain top-16 (no forced blocks), w=512, bf16.  The same inputs with the
initial and two local blocks forced among the 16 are timed beside it
(``c3_forced``).

Prints ONE JSON line (rank 0): the metric, tokens/s, the dominant kernel's
roofline (algorithmic work / its HIP-event-timed launch duration, bound set
from its measured HBM bytes), the forward and backward timed apart (medians
of 20 after 5 warm-up steps), per-kernel MFMA fractions, the decode step
(one new query per sequence against 32K caches, B=32 and B=1: tokens/s and
HBM fraction), the compression phi's forward / backward time, and CPU baselines (the float32 CPU oracle on a bounded row
sample of c3, and dense on c1).  ``--workload dec|dec_b1|dec_c5|c4|c5`` runs
one of the other workloads alone.
"""

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "openbox-llm_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "NSA fused fwd+bwd tokens/s at T=32K bf16; % of MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2500.0
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

# geometry tuples: (cmp_block, cmp_stride, sel_block, n_sel, window, force_init, n_local)
WORKLOADS = {
    "c3": dict(kind="fused", B=1, T=32768, Hq=64, Hkv=4, D=128, geom=(32, 16, 64, 16, 512, False, 0),
               head_scale=True, in_scale=1.0,
               desc="BASELINE config 3: fused 3-branch NSA fwd+bwd, B1 T32768 Hq64 Hkv4 D128, "
                    "l32/d16 l'64 top-16 w512, bf16"),
    "c3_forced": dict(kind="fused", B=1, T=32768, Hq=64, Hkv=4, D=128, geom=(32, 16, 64, 16, 512, True, 2),
                      head_scale=True, in_scale=1.0,
                      desc="config 3 with the initial block and 2 local blocks forced among the top-16"),
    "c2": dict(kind="selection", B=4, T=8192, Hq=16, Hkv=1, D=64, geom=(32, 16, 64, 16, 512, False, 0),
               head_scale=False, in_scale=1.0,
               desc="BASELINE config 2: selection branch only, fwd+bwd, B4 T8192 Hq16 Hkv1 D64, l'64 top-16, "
                    "indices from compression importance (l32/d16), bf16"),
    "c1": dict(kind="fused", B=1, T=1024, Hq=4, Hkv=1, D=64, geom=(32, 16, 64, 16, 512, True, 2),
               head_scale=False, in_scale=0.125,
               desc="BASELINE config 1 shape: B1 T1024 Hq4 Hkv1 D64, l32/d16 l'64 top-16 (init + 2 local) w512"),
    "small": dict(kind="fused", B=1, T=4096, Hq=16, Hkv=1, D=128, geom=(32, 16, 64, 16, 512, False, 0),
                  head_scale=True, in_scale=1.0, desc="reduced c3-like shape for quick checks"),
    "c4": dict(kind="model", B=8, T=4096, Hq=12, Hkv=2, D=64, geom=(32, 16, 64, 16, 512, False, 0),
               vocab=32000, d_model=768, n_layers=12, ffn_hidden=2048,
               desc="BASELINE config 4: 12-layer d768 decoder (12q/2kv heads, hd64, SwiGLU 2048, RMSNorm, RoPE 1e4, "
                    "vocab 32000), NSA l32/d16 l'64 top-16 w512 in every layer, bf16 autocast AdamW step, 8x4096 "
                    "tokens; dense arms: the same model with causal SDPA attention, and with the reference's "
                    "materialised causal score matrix"),
    "dec": dict(kind="decode", B=32, T=32768, Hq=64, Hkv=4, D=128, geom=(32, 16, 64, 16, 512, False, 0),
                desc="decode step (nsa_decode_fwd): 32 sequences, one new query each at position 32767 of "
                     "32K-token caches, config-3 heads (Hq64 Hkv4 D128) and geometry (l32/d16 l'64 top-16 w512), bf16"),
    "dec_b1": dict(kind="decode", B=1, T=32768, Hq=64, Hkv=4, D=128, geom=(32, 16, 64, 16, 512, False, 0),
                   desc="decode step, one sequence (latency): as dec with B=1"),
    "dec_c5": dict(kind="decode", B=4, T=131072, Hq=32, Hkv=2, D=128, geom=(32, 16, 64, 32, 512, False, 0),
                   desc="decode step, 4 sequences at 128K with config-5 heads (Hq32 Hkv2 D128, top-32)"),
    "c5": dict(kind="forward", B=1, T=131072, Hq=32, Hkv=2, D=128, geom=(32, 16, 64, 32, 512, False, 0),
               head_scale=False, in_scale=1.0, shift_frac=0.01, shift=3.0,
               desc="BASELINE config 5: NSA forward only, B1 T131072 Hq32 Hkv2 D128, l32/d16 l'64 top-32 w512, bf16, "
                    "1% of the 64-token key blocks shifted by +3 sigma"),
}

# HBM bytes per launch of a kernel, measured with two rocprofv3 PMC passes of
# this bench (FETCH_SIZE, then WRITE_SIZE) and scaled by what the same
# counters read for a plain 1 GiB device copy (x2.0 and x1.0); the commands
# and counter values are kept under profiles/.  Keyed by (workload, kernel).
MEASURED_TRAFFIC = {   # profiles/nsa_fused_c3_pmc_traffic.md: bytes read + bytes written per launch
    ("c3", "dkdv[sel]"): 1.740e10 + 8.803e9,
    ("c3", "fwd[sel]"): 8.435e9 + 8.733e9,
    ("c3", "dq[cmp+win]"): 1.131e10 + 5.369e8,
    ("c3", "fwd[win]"): 1.003e10 + 1.663e9,
    ("c3", "dkdv[win]"): 1.007e10 + 1.384e8,
    ("c3", "dkdv[cmp]"): 2.739e9 + 1.892e8,
    ("c3", "fwd[cmp]"): 6.543e8 + 1.420e9,
    ("c3", "nsa_bwd_prep"): 2.273e9 + 8.012e8,
    ("c3", "nsa_importance_topn"): 6.019e8 + 2.509e8,
    ("c3", "nsa_pool_fwd"): 5.853e7 + 2.096e6,
}

ISO_STEPS = 2   # untimed steps with every call timed (per-kernel spans, dominant kernel)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(w, dev, dtype, seed=0):
    """Seeded synthetic inputs of a workload, generated on `dev`: q, kc, vc,
    ks, vs, kw, vw ~ N(0,1) * in_scale (times a per-head U(0.5, 2) scale when
    `head_scale`), gate logits N(0,1), dO N(0,1)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    B, T, Hq, Hkv, D = w["B"], w["T"], w["Hq"], w["Hkv"], w["D"]

    def rn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)

    q = rn(B, Hq, T, D) * w["in_scale"]
    kv = [rn(B, Hkv, T, D) * w["in_scale"] for _ in range(6)]
    if w["head_scale"]:
        sq = torch.rand(Hq, generator=g, device=dev) * 1.5 + 0.5
        skv = torch.rand(6, Hkv, generator=g, device=dev) * 1.5 + 0.5
        q = q * sq[None, :, None, None]
        kv = [x * skv[i][None, :, None, None] for i, x in enumerate(kv)]
    if w.get("shift_frac"):
        # a seeded 1% of the 64-token key blocks get a mean shift on every key
        # of every branch: peaked block scores for the top-n
        nb = T // 64
        pick = torch.randperm(nb, generator=g, device=dev)[:max(1, round(w["shift_frac"] * nb))]
        tok = (pick[:, None] * 64 + torch.arange(64, device=dev)[None, :]).reshape(-1)
        for i in (0, 2, 4):
            kv[i][:, :, tok] += w["shift"]
    gate = rn(B, Hq, T, 3)
    do = rn(B, Hq, T, D)
    ins = [t.to(dtype).contiguous() for t in [q] + kv + [gate]]
    return ins, do.to(dtype).contiguous()


def keys_visible(w, idx):
    """(sum_win, sum_cmp, sum_sel) visible keys over all (b, hkv, t) rows of one head."""
    T = w["T"]
    l, d, ls, n, win, _, _ = w["geom"]
    t = torch.arange(T, device=idx.device, dtype=torch.int64)
    k_win = torch.clamp(t + 1, max=win).sum() * w["B"] * w["Hkv"]
    n_cmp = (T - l) // d + 1 if T >= l else 0
    k_cmp = torch.where(t >= l - 1, torch.clamp((t - l + 1) // d + 1, max=n_cmp), torch.zeros_like(t))
    k_cmp = k_cmp.sum() * w["B"] * w["Hkv"]
    bl = idx.long()
    start = bl * ls
    vis = torch.clamp(torch.minimum(t[None, None, :, None] + 1, start + ls) - start, min=0)
    vis = torch.where(bl >= 0, vis, torch.zeros_like(vis))
    return int(k_win), int(k_cmp), int(vis.sum())


def sel_pairs(w, idx):
    """(query, selected block) pairs with a visible key: the CSR length."""
    ls = w["geom"][2]
    t = torch.arange(w["T"], device=idx.device, dtype=torch.int64)[None, None, :, None]
    bl = idx.long()
    return int(((bl >= 0) & (bl * ls <= t)).sum())


def kernel_flops(w, kv):
    """Algorithmic FLOPs of one launch of each timed library call (span name -> flops).

    Per (query head, visible key): forward 4*D (QK^T and PV); range dK/dV
    kernels 8*D (S, dP, dV, dK); range dQ kernels 2*D (dQ only: their S and
    dP are recomputed work, counted once in the dK/dV kernel).  The selection
    dK/dV kernel also forms the dQ partials (10*D).  Every branch sums to
    14*D per key, the fwd+bwd convention of the metric.  ``dq[cmp+win]`` is
    the one launch that computes both range dQs; the per-branch ``dq[cmp]`` /
    ``dq[win]`` entries describe the unfused path and are not added to it.
    """
    G = w["Hq"] // w["Hkv"]
    D = w["D"]
    k_win, k_cmp, k_sel = kv
    out = {}
    for br, k in (("win", k_win), ("cmp", k_cmp), ("sel", k_sel)):
        rows_keys = k * G
        out[f"fwd[{br}]"] = 4 * D * rows_keys
        if br == "sel":
            out["dkdv[sel]"] = 10 * D * rows_keys
        else:
            out[f"dq[{br}]"] = 2 * D * rows_keys
            out[f"dkdv[{br}]"] = 8 * D * rows_keys
    out["dq[cmp+win]"] = out["dq[cmp]"] + out["dq[win]"]
    return out


def step_flops(w, kv):
    """Algorithmic FLOPs of one fwd+bwd step: 14*D per (query head, visible key)."""
    G = w["Hq"] // w["Hkv"]
    ks = kv if w["kind"] == "fused" else (0, 0, kv[2])
    return 14 * w["D"] * G * sum(ks)


def sel_dkdv_bytes(w, pairs):
    """Bytes the block-outer selection dK/dV schedule must move per launch,
    with perfect caching inside one work item: per (query, block) pair the G
    query rows of Q and dO and the dQ partial written (3*G*D elements) plus
    the row statistics (2*G float); per selection block K, V and K^T read
    once and dK, dV written in float32.  And the compulsory bytes: every
    tensor the kernel touches once."""
    B, T, Hkv, D = w["B"], w["T"], w["Hkv"], w["D"]
    G = w["Hq"] // Hkv
    e = 2
    per_pair = 3 * G * D * e + 2 * G * 4
    keys = B * Hkv * T
    per_key = 3 * D * e + 2 * D * 4
    algorithmic = pairs * per_pair + keys * per_key
    rows = B * w["Hq"] * T
    compulsory = 3 * rows * D * e + 2 * rows * 4 + keys * per_key
    return algorithmic, compulsory


def compulsory_bytes(w, kernel, kv, pairs):
    """Bytes a kernel must move at least: every tensor of its operation read or
    written once (inputs at their sizes, outputs once per row), or None where
    no formula is kept.  The selection dK/dV: Q, dO and dQ rows (one per query
    row), the row statistics, and per key K, V, K^T read and dK, dV written in
    float32."""
    if kernel == "dkdv[sel]":
        return sel_dkdv_bytes(w, pairs)[1]
    return None


def roofline_of(w, name, flops, per_launch_s, traffic, kv, pairs):
    """Roofline entry of one kernel: the bound is set by its arithmetic
    intensity over its compulsory bytes against the ridge point of the peaks
    (bf16 MFMA FLOP/s over HBM B/s); `frac` is the algorithmic work per launch
    (FLOPs, or the compulsory bytes when HBM-bound) / launch duration / peak.
    `traffic` is the counter-measured HBM bytes per launch and
    `traffic_ratio` its multiple of the compulsory bytes."""
    tflops = flops / per_launch_s / 1e12
    comp = compulsory_bytes(w, name, kv, pairs)
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    ent = {"kernel": name, "launch_ms": round(per_launch_s * 1e3, 4), "algorithmic_tflop": round(flops / 1e12, 4),
           "traffic": traffic, "compulsory_bytes": comp}
    hbm_frac = comp / per_launch_s / 1e9 / PEAK_HBM_GBS if comp else None
    intensity = flops / comp if comp else None
    if intensity is None or intensity >= ridge:
        ent.update({"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(tflops / PEAK_BF16_TFLOPS, 4)})
    else:
        gbs = comp / per_launch_s / 1e9
        ent.update({"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4)})
    ent.update({"mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                "hbm_frac": round(hbm_frac, 4) if hbm_frac is not None else None,
                "intensity_flop_per_byte": round(intensity, 1) if intensity else None,
                "ridge_flop_per_byte": round(ridge, 1)})
    if traffic:
        ent["measured_gbs"] = round(traffic / per_launch_s / 1e9, 1)
        ent["traffic_ratio"] = round(traffic / comp, 2) if comp else None
    if name == "dkdv[sel]":
        # the bytes of its block-outer schedule (Q, dO and dQ-partial rows per
        # (query, block) pair): what the kernel can move at best as built
        sched = sel_dkdv_bytes(w, pairs)[0]
        ent["schedule_bytes"] = sched
        ent["achieved_gbs"] = round(sched / per_launch_s / 1e9, 1)
    return ent


def _setup(w, dev, dtype, seed=0):
    import nsa_hip_ops as ops
    geom = ops.NSAGeometry(*w["geom"])
    ins, do = make_inputs(w, dev, dtype, seed)
    return geom, ins, do


def make_step(w, geom, ins, do):
    """One fwd+bwd step of the workload -> block indices of the step."""
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    import nsa_selection_backward as nsb

    if w["kind"] == "fused":
        xs = [t.requires_grad_() for t in ins]

        def fwd():
            for x in xs:
                x.grad = None
            return nfk.nsa_attention(*xs, geom)

        def step():
            out, idx = fwd()
            out.backward(do)
            return idx
        step.fwd = lambda: fwd()[0]
        step.bwd = lambda out: out.backward(do)
        return step
    # selection only: indices from the compression importance (computed once;
    # they are an input of the selection kernels), keys/values of the
    # selection branch
    q, kc, ks, vs = ins[0], ins[1], ins[3], ins[4]
    with torch.no_grad():
        k_cmp = ops.pool_fwd(kc, geom.cmp_block, geom.cmp_stride)
        _, lse_c = ops.range_fwd(ops.MODE_COMPRESS, q, k_cmp, k_cmp, 0, geom.cmp_block, geom.cmp_stride)
        idx = ops.importance_topn(q, k_cmp, lse_c, geom)
    xs = [t.requires_grad_() for t in (q, ks, vs)]

    def fwd():
        for x in xs:
            x.grad = None
        return nsb.selection_attn_triton(*xs, idx, geom.sel_block)

    def step():
        fwd().backward(do)
        return idx
    step.fwd = fwd
    step.bwd = lambda out: out.backward(do)
    return step


def run_gpu(args, w, name):
    import nsa_hip_ops as ops

    dev = torch.device("cuda:0")
    geom, ins, do = _setup(w, dev, torch.bfloat16)
    step = make_step(w, geom, ins, do)
    log(f"[bench] {name}: warmup {args.warmup} step(s) on {torch.cuda.get_device_name(0)}")
    idx = None
    for _ in range(args.warmup):
        idx = step()
    torch.cuda.synchronize()
    if idx is None:
        idx = step()
        torch.cuda.synchronize()
    kv = keys_visible(w, idx)
    pairs = sel_pairs(w, idx)
    flops_of = kernel_flops(w, kv)
    # untimed, first: every call timed (the backward runs in order on one
    # stream), so that each kernel's duration is its own; picks the dominant
    # kernel
    iso = ops.LaunchTimer()
    try:
        ops.set_timer(iso)
        for _ in range(ISO_STEPS):
            step()
        torch.cuda.synchronize()
    finally:
        ops.set_timer(None)
    iso_spans = iso.summary_ms()
    modeled = {k: v for k, v in iso_spans.items() if k in flops_of}
    dom = max(modeled, key=lambda k: modeled[k][1]) if modeled else None
    # timed: HIP events around the dominant kernel's calls only
    timer = ops.LaunchTimer(only=[dom] if dom else [])
    ops.set_timer(timer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ops.set_timer(None)
    ms = (t1 - t0) * 1e3 / args.steps
    # forward and backward apart (not the headline: that is the timed steps above)
    split = time_fwd_bwd(step)
    # peak device memory of one step (inputs resident, as in the timed steps)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    torch.cuda.synchronize()
    mem = {"peak_gib": round(torch.cuda.max_memory_allocated() / 2**30, 3),
           "peak_above_inputs_gib": round((torch.cuda.max_memory_allocated() - base) / 2**30, 3)}
    return dict(ms=ms, spans=timer.summary_ms(), iso_spans=iso_spans, dom=dom, flops_of=flops_of, kv=kv,
                pairs=pairs, ins=ins, do=do, idx=idx, split=split, geom=geom, mem=mem)


def time_fwd_bwd(step, warmup=5, reps=20):
    """Forward and backward of a step timed apart with HIP events around each
    call, medians of `reps` after `warmup` steps -> dict (ms)."""
    for _ in range(warmup):
        step.bwd(step.fwd())
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(reps)]
    for e in ev:
        e[0].record()
        out = step.fwd()
        e[1].record()
        step.bwd(out)
        e[2].record()
    torch.cuda.synchronize()
    f = [e[0].elapsed_time(e[1]) for e in ev]
    b = [e[1].elapsed_time(e[2]) for e in ev]
    t = [e[0].elapsed_time(e[2]) for e in ev]
    return {"fwd_ms": round(statistics.median(f), 3), "bwd_ms": round(statistics.median(b), 3),
            "fwd_bwd_ms": round(statistics.median(t), 3), "warmup": warmup, "reps": reps,
            "note": "HIP events around each call, medians"}


def time_gpu_only(args, w, name):
    """Timed steps of a workload, no per-call spans: ms per step."""
    dev = torch.device("cuda:0")
    geom, ins, do = _setup(w, dev, torch.bfloat16)
    step = make_step(w, geom, ins, do)
    for _ in range(max(1, args.warmup)):
        idx = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    log(f"[bench] {name}: {ms:.3f} ms per step")
    return ms, keys_visible(w, idx)


def run_cpu_baseline(w, ins_dev, do_dev, rows_n, threads):
    """The float32 CPU oracle on `rows_n` evenly spaced query rows of the
    same inputs (copied from the GPU; only the sampled query rows of q, gate
    and dO are needed, the keys and values are copied whole)."""
    from oracle import nsa_oracle as O

    torch.set_num_threads(threads)
    B, T, Hq, Hkv, D = w["B"], w["T"], w["Hq"], w["Hkv"], w["D"]
    l, d, ls, n, win, fi, nl = w["geom"]
    cfg = O.NSAConfig(l, d, ls, n, win, fi, nl)
    rows = torch.linspace(0, T - 1, rows_n).round().long().unique()
    rows_dev = rows.to(do_dev.device)
    q = torch.zeros(B, Hq, T, D)
    q[:, :, rows] = ins_dev[0].detach()[:, :, rows_dev].float().cpu()
    gate = torch.zeros(B, Hq, T, 3)
    gate[:, :, rows] = ins_dev[7].detach()[:, :, rows_dev].float().cpu()
    do = torch.zeros(B, Hq, T, D)
    do[:, :, rows] = do_dev[:, :, rows_dev].float().cpu()
    ins = [q] + [t.detach().float().cpu() for t in ins_dev[1:7]] + [gate]
    chunk = 16
    n_slc = T // ls
    S = min(n, n_slc)
    t0 = time.perf_counter()
    xs = [t.clone().requires_grad_() for t in ins]
    k_cmp = O.pool_mean(xs[1], l, d)
    v_cmp = O.pool_mean(xs[2], l, d)
    for c0 in range(0, rows.numel(), chunk):
        r = rows[c0:c0 + chunk]
        with torch.no_grad():
            imp = O.importance_rows(xs[0].detach(), k_cmp.detach(), cfg, r, T)
            sel = O.topn_from_scores(O.selection_scores(imp, cfg, t_pos=r), S)
        idx = torch.full((B, Hkv, T, S), -1, dtype=torch.int32)
        idx[:, :, r] = sel
        out, _ = O.nsa_rows(*xs, idx, cfg, r, k_cmp=k_cmp, v_cmp=v_cmp)
        (out * do[:, :, r]).sum().backward(retain_graph=True)
    t1 = time.perf_counter()
    secs = t1 - t0
    return rows.numel() * B / secs, secs, rows.numel()


def run_cpu_c1(threads, reps=3):
    """Config 1 on the CPU: the dense float32 oracle (importance, top-n and
    the three gated branches, forward + backward), median of `reps` runs
    after one warm-up, for the extended geometry (l32/d16/l'64, init + 2
    local forced) and the aligned l = d = l' = 64 grid with no forcing
    (exactly the reference path).  -> {variant: (tokens/s, median s)}."""
    from oracle import nsa_oracle as O

    torch.set_num_threads(threads)
    w = WORKLOADS["c1"]
    ins, do = make_inputs(w, torch.device("cpu"), torch.float32)
    res = {}
    for variant, cfg in (("extended", O.NSAConfig(*w["geom"])), ("aligned64", O.NSAConfig.reference(64, 16, 512))):
        times = []
        for r in range(reps + 1):
            xs = [t.clone().requires_grad_() for t in ins]
            t0 = time.perf_counter()
            out, _ = O.nsa_forward_reference(*xs, cfg)
            out.backward(do)
            dt = time.perf_counter() - t0
            if r > 0:
                times.append(dt)
        med = statistics.median(times)
        res[variant] = (w["B"] * w["T"] / med, med)
    return res


def time_gpu_c1(reps=20):
    """Config 1 on the GPU in float32 (the CPU baseline's precision): ms per
    fwd+bwd step, extended and aligned-64 geometry."""
    import nsa_hip_ops as ops
    w = WORKLOADS["c1"]
    dev = torch.device("cuda:0")
    ins, do = make_inputs(w, dev, torch.float32)
    res = {}
    for variant, geom in (("extended", ops.NSAGeometry(*w["geom"])),
                          ("aligned64", ops.NSAGeometry.aligned(64, 16, 512))):
        xs = [t.clone().requires_grad_() for t in ins]

        def step():
            for x in xs:
                x.grad = None
            out, _ = ops.nsa_attention(*xs, geom)
            out.backward(do)
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            step()
        torch.cuda.synchronize()
        res[variant] = (time.perf_counter() - t0) * 1e3 / reps
    return res


def run_model_bench(args, w, arms=("nsa", "dense", "dense_ref")):
    """Config 4: one bf16-autocast AdamW training step of the decoder, NSA
    (fused HIP attention) against the same model with dense causal attention
    -- through SDPA's flash kernels ("dense"), and as the reference's own
    control arm computes it, the full causal score matrix materialised
    (FullAttention, nsa_model.py:377-419: "dense_ref", the arm of the
    reference's memory claim); tokens/s and peak device memory per arm."""
    import nsa_model
    dev = torch.device("cuda:0")
    B, T = w["B"], w["T"]
    l, d, ls, n, win, fi, nl = w["geom"]
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randint(0, w["vocab"], (B, T), generator=g, device=dev)
    y = torch.randint(0, w["vocab"], (B, T), generator=g, device=dev)
    out = {}
    for arm in arms:
        torch.cuda.empty_cache()
        base = torch.cuda.memory_allocated()   # other workloads' tensors still held by the caller
        torch.manual_seed(0)
        m = nsa_model.NSATransformer(
            vocab_size=w["vocab"], d_model=w["d_model"], n_layers=w["n_layers"], n_q_heads=w["Hq"],
            n_kv_heads=w["Hkv"], max_seq_len=T, ffn_hidden=w["ffn_hidden"], norm="rms", ffn="swiglu", pos="rope",
            tie_embeddings=False, attn_type="nsa" if arm == "nsa" else "full", attn_impl="fused",
            dense_impl="ref" if arm == "dense_ref" else "sdpa",
            block_size=l, cmp_stride=d, sel_block=ls, n_selected_blocks=n, window=win, force_init=fi,
            n_local=nl).to(dev)
        opt = torch.optim.AdamW(m.parameters(), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
        losses = []

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                _, loss = m(x, y)
            opt.zero_grad(set_to_none=True)
            loss.backward()
            opt.step()
            return loss
        for _ in range(max(1, args.warmup)):
            losses.append(float(step()))
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        steps = min(args.steps, 3) if arm == "dense_ref" else args.steps   # ~0.3 s a step
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        losses.append(float(loss))
        out[arm] = {"ms_per_step": round(ms, 2), "tokens_per_s": round(B * T / (ms / 1e3), 1),
                    "peak_mem_gib": round((torch.cuda.max_memory_allocated() - base) / 2**30, 2),
                    "params_m": round(sum(p.numel() for p in m.parameters()) / 1e6, 2),
                    "loss_first_last": [round(losses[0], 4), round(losses[-1], 4)]}
        log(f"[bench] c4 {arm}: {ms:.1f} ms per step, peak {out[arm]['peak_mem_gib']} GiB")
        del m, opt
    return out


def run_forward_bench(args, w, name):
    """Config 5: the NSA forward alone (pooling, compression, importance /
    top-n, selection, window, gate), no autograd; per-call spans for the
    roofline of its dominant kernel."""
    import nsa_hip_ops as ops
    dev = torch.device("cuda:0")
    geom, ins, _ = _setup(w, dev, torch.bfloat16)

    def step():
        with torch.no_grad():
            return ops.nsa_attention(*ins, geom)
    for _ in range(max(1, args.warmup)):
        _, idx = step()
    torch.cuda.synchronize()
    kv = keys_visible(w, idx)
    iso = ops.LaunchTimer()
    ops.set_timer(iso)
    for _ in range(ISO_STEPS):
        step()
    torch.cuda.synchronize()
    ops.set_timer(None)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    G, D = w["Hq"] // w["Hkv"], w["D"]
    fwd_flops = {f"fwd[{br}]": 4 * D * G * k for br, k in zip(("win", "cmp", "sel"), kv)}
    spans = iso.summary_ms()
    return {"ms_per_step": round(ms, 3), "tokens_per_s": round(w["B"] * w["T"] / (ms / 1e3), 1),
            "fwd_tflop": round(sum(fwd_flops.values()) / 1e12, 3),
            "mfu": round(sum(fwd_flops.values()) / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "visible_keys": {"win": kv[0], "cmp": kv[1], "sel": kv[2]},
            "per_kernel": per_kernel_table(spans, fwd_flops, PEAK_BF16_TFLOPS, name)}


def run_decode_bench(w, steps=200, warmup=10):
    """One decode step per sequence (nsa_decode_fwd) on caches resident in
    HBM, timed with HIP events over ``steps`` calls.  Algorithmic bytes: every
    visible cache row read once (pooled tokens, window keys, keys of the
    picked blocks; K and V) plus q, gate and out."""
    import nsa_hip_ops as ops
    dev = torch.device("cuda:0")
    geom = ops.NSAGeometry(*w["geom"])
    B, Hq, Hkv, D, T = w["B"], w["Hq"], w["Hkv"], w["D"], w["T"]
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, Hq, D, device=dev, generator=g).bfloat16()
    gate = torch.randn(B, Hq, 3, device=dev, generator=g).bfloat16()
    caches = [torch.randn(B, Hkv, T, D, device=dev, generator=g).bfloat16() for _ in range(6)]
    k_cmp = ops.pool_fwd(caches[0], geom.cmp_block, geom.cmp_stride)
    v_cmp = ops.pool_fwd(caches[1], geom.cmp_block, geom.cmp_stride)
    lens = torch.full((B,), T, dtype=torch.int32, device=dev)
    ws = torch.empty(ops.decode_workspace_bytes(B, Hq, Hkv, D, T, k_cmp.shape[2], geom), device=dev,
                     dtype=torch.uint8)

    def step():
        return ops.decode_fwd(q, k_cmp, v_cmp, *caches[2:], gate, lens, geom, workspace=ws)
    for _ in range(warmup):
        out, idx = step()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        step()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps
    t = T - 1
    nvis = (t + 1 - geom.cmp_block) // geom.cmp_stride + 1
    ls = geom.sel_block
    sel_keys = 0
    for j in idx.flatten().tolist():
        if j >= 0:
            sel_keys += max(0, min((j + 1) * ls, t + 1) - j * ls)
    kv_rows = B * Hkv * (nvis + min(geom.window, T)) + sel_keys
    alg = kv_rows * 2 * D * 2 + B * Hq * (2 * D + 3) * 2
    gbs = alg / (us / 1e6) / 1e9
    return {"us_per_step": round(us, 2), "tokens_per_s": round(B / (us / 1e6), 1), "steps": steps,
            "algorithmic_bytes": alg, "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "workspace_bytes": ws.numel(), "desc": w["desc"]}


def run_phi_bench(reps=20):
    """The NSA paper's compression phi (``nsa_hip_ops.phi_compress``) on the
    config-3 keys of one layer: B1 Hkv4 T32768 D128, span 32 stride 16,
    hidden 128, bf16; forward and backward timed with HIP events."""
    import nsa_hip_ops as ops
    dev = torch.device("cuda:0")
    B, H, T, D, Hd, l, d = 1, 4, 32768, 128, 128, 32, 16
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(B, H, T, D, device=dev, generator=g).bfloat16().requires_grad_()
    params = [(0.3 * torch.randn(l, D, device=dev, generator=g)).requires_grad_(),
              (torch.randn(Hd, l * D, device=dev, generator=g) / 64).requires_grad_(),
              torch.zeros(Hd, device=dev, requires_grad=True),
              (torch.randn(D, Hd, device=dev, generator=g) / 11).requires_grad_(),
              torch.zeros(D, device=dev, requires_grad=True)]
    n = (T - l) // d + 1
    dout = torch.randn(B, H, n, D, device=dev, generator=g).bfloat16()
    for _ in range(3):
        ops.phi_compress(x, *params, l, d).backward(dout)
    torch.cuda.synchronize()
    a, b, c = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    outs = []
    a.record()
    for _ in range(reps):
        outs.append(ops.phi_compress(x, *params, l, d))
    b.record()
    for y in outs:
        y.backward(dout)
    c.record()
    torch.cuda.synchronize()
    fwd_ms, bwd_ms = a.elapsed_time(b) / reps, b.elapsed_time(c) / reps
    flops = B * H * n * (l * D * Hd + Hd * D) * 2
    return {"fwd_us": round(fwd_ms * 1e3, 1), "bwd_us": round(bwd_ms * 1e3, 1),
            "fwd_tflops": round(flops / fwd_ms / 1e9, 1), "fwd_mfma_frac": round(flops / fwd_ms / 1e9 / PEAK_BF16_TFLOPS, 4),
            "shape": "B1 Hkv4 T32768 D128, l32 d16, hidden 128, bf16 (one of the two compressors of a config-3 layer)"}


def run_other_configs(args):
    """The other BASELINE configs beside the c3 line: c2 (selection branch
    fwd+bwd), c5 (long-context forward) and c4 (the 150M training step, NSA
    against dense attention, time and peak memory of each arm)."""
    small = argparse.Namespace(steps=min(args.steps, 10), warmup=min(args.warmup, 3))
    out = {}
    w2 = WORKLOADS["c2"]
    ms2, kv2 = time_gpu_only(small, w2, "c2")
    f2 = step_flops(w2, kv2)
    out["c2"] = {"ms_per_step": round(ms2, 3), "tokens_per_s": round(w2["B"] * w2["T"] / (ms2 / 1e3), 1),
                 "tflop": round(f2 / 1e12, 4), "mfma_frac": round(f2 / (ms2 / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                 "desc": w2["desc"]}
    torch.cuda.empty_cache()
    c5 = run_forward_bench(small, WORKLOADS["c5"], "c5")
    out["c5"] = {k: c5[k] for k in ("ms_per_step", "tokens_per_s", "fwd_tflop", "mfu")}
    out["c5"]["desc"] = WORKLOADS["c5"]["desc"]
    torch.cuda.empty_cache()
    c4 = run_model_bench(small, WORKLOADS["c4"])
    c4["nsa_vs_dense_time"] = round(c4["dense"]["ms_per_step"] / c4["nsa"]["ms_per_step"], 4)
    c4["nsa_vs_dense_memory"] = round(c4["nsa"]["peak_mem_gib"] / c4["dense"]["peak_mem_gib"], 4)
    c4["nsa_vs_dense_ref_time"] = round(c4["dense_ref"]["ms_per_step"] / c4["nsa"]["ms_per_step"], 4)
    c4["nsa_vs_dense_ref_memory"] = round(c4["nsa"]["peak_mem_gib"] / c4["dense_ref"]["peak_mem_gib"], 4)
    c4["desc"] = WORKLOADS["c4"]["desc"]
    # the same model and tokens per step at 4x the sequence length (B2 x
    # 16384): dense attention's work per token grows with T, NSA's stays near
    # its top-n and window budget (no materialised arm: its score matrices
    # would not fit)
    torch.cuda.empty_cache()
    c4l = run_model_bench(small, dict(WORKLOADS["c4"], B=2, T=16384), arms=("nsa", "dense"))
    c4l["nsa_vs_dense_time"] = round(c4l["dense"]["ms_per_step"] / c4l["nsa"]["ms_per_step"], 4)
    c4l["nsa_vs_dense_memory"] = round(c4l["nsa"]["peak_mem_gib"] / c4l["dense"]["peak_mem_gib"], 4)
    c4l["desc"] = "config 4's model and step at B2 x T16384 (the same 32768 tokens a step)"
    c4["long_context"] = c4l
    out["c4"] = c4
    torch.cuda.empty_cache()
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def per_kernel_table(iso_spans, flops_of, peak, workload):
    """name -> {ms per step, calls per step, algorithmic TFLOP per launch,
    MFMA fraction, and where the PMC traffic was measured for this workload,
    HBM GB/s and fraction of the HBM peak}."""
    out = {}
    for name, (calls, tot) in sorted(iso_spans.items(), key=lambda x: -x[1][1]):
        ent = {"ms_per_step": round(tot / ISO_STEPS, 4), "calls_per_step": calls // ISO_STEPS}
        per = tot / calls / 1e3 if calls > 0 else None
        if name in flops_of and per:
            ent["tflop_per_launch"] = round(flops_of[name] / 1e12, 4)
            ent["mfma_frac"] = round(flops_of[name] / per / 1e12 / peak, 4)
        traffic = MEASURED_TRAFFIC.get((workload, name))
        if traffic and per:
            ent["hbm_gbs"] = round(traffic / per / 1e9, 1)
            ent["hbm_frac"] = round(traffic / per / 1e9 / PEAK_HBM_GBS, 4)
        out[name] = ent
    return out


def measure_branches(w, geom, ins, do, kv, reps=2):
    """Each branch's work as launches of its own, so that every launch is one
    branch: the forward through the per-branch calls (compression; selection
    partials, then their merge as its own launch; the window alone; the gate
    blend), the backward with one dQ launch per branch
    (``FUSE_RANGE_DQ = False``, ``SEPARATE_SEL_DQ = True``).  The timed step
    fuses these launches (the merge and the gate into the window forward, the
    three dQs into one launch); this split only attributes time to branches.
    Per branch: its launches (ms per step), their sum, the branch's
    algorithmic FLOPs (14 D per visible (query head, key), fwd + bwd) and the
    MFMA fraction; the gate blend and the backward's row statistics are
    reported as `gate`."""
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops
    q, kc, vc, ks, vs, kw, vw, gate = (t.detach() for t in ins)
    Hkv = ks.shape[1]
    fwd = ops.LaunchTimer()
    ops.set_timer(fwd)
    try:
        with torch.no_grad():
            for _ in range(reps):
                k_cmp = ops.pool_fwd(kc, geom.cmp_block, geom.cmp_stride)
                v_cmp = ops.pool_fwd(vc, geom.cmp_block, geom.cmp_stride)
                o_c, lse_c = ops.range_fwd(ops.MODE_COMPRESS, q, k_cmp, v_cmp, 0, geom.cmp_block, geom.cmp_stride)
                idx = ops.importance_topn(q, k_cmp, lse_c, geom)
                parts, _ = ops.sel_fwd_partials(q, ks, vs, idx, geom.sel_block)
                o_s, _ = ops.sel_merge(idx, parts, q.shape, Hkv, geom.sel_block)
                del parts
                o_w, _ = ops.range_fwd(ops.MODE_WINDOW, q, kw, vw, geom.window)
                ops.gate_fwd(gate, o_c, o_s, o_w)
        torch.cuda.synchronize()
    finally:
        ops.set_timer(None)
    saved = (ops.FUSE_RANGE_DQ, ops.SEPARATE_SEL_DQ)
    bwd_names = ["dq[win]", "dq[cmp]", "dq[sel]", "dkdv[sel]", "dkdv[win]", "dkdv[cmp]", "nsa_bwd_prep"]
    bwd = ops.LaunchTimer(only=bwd_names)
    ops.FUSE_RANGE_DQ, ops.SEPARATE_SEL_DQ = False, True
    try:
        xs = [t.requires_grad_() for t in (q, kc, vc, ks, vs, kw, vw, gate)]
        for i in range(reps + 1):
            out, _ = nfk.nsa_attention(*xs, geom)
            if i > 0:
                ops.set_timer(bwd)
            out.backward(do)
            ops.set_timer(None)
            del out
        torch.cuda.synchronize()
    finally:
        ops.set_timer(None)
        ops.FUSE_RANGE_DQ, ops.SEPARATE_SEL_DQ = saved
        for t in (q, kc, vc, ks, vs, kw, vw, gate):
            t.requires_grad_(False)
            t.grad = None
    spans = {**{k: v for k, v in fwd.summary_ms().items()}, **bwd.summary_ms()}
    G, D = w["Hq"] // w["Hkv"], w["D"]
    k_win, k_cmp_n, k_sel = kv

    def branch(names, keys):
        launches = {n: round(spans[n][1] / reps, 4) for n in names if n in spans}
        ms = sum(launches.values())
        ent = {"launches_ms": launches, "ms_per_step": round(ms, 4)}
        if keys is not None:
            flops = 14 * D * G * keys
            ent.update({"tflop": round(flops / 1e12, 4),
                        "mfma_frac": round(flops / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4) if ms > 0 else None})
        return ent
    return {
        "selection": branch(["fwd[sel]", "nsa_sel_merge", "dkdv[sel]", "dq[sel]"], k_sel),
        "window": branch(["fwd[win]", "dq[win]", "dkdv[win]"], k_win),
        "compression": branch(["fwd[cmp]", "dq[cmp]", "dkdv[cmp]"], k_cmp_n),
        "gate": branch(["nsa_gate_fwd", "nsa_bwd_prep"], None),
        "note": "each branch's launches run apart (merge, gate and dQs unfused) in an untimed pass; "
                "mfma_frac = 14 D per visible (query head, key) / their summed time / 2.5 PFLOP/s",
    }


def branch_fractions(iso_spans, flops_of, peak):
    """MFMA fraction of the fused step's launches grouped by branch.
    selection = fwd[sel] + dkdv[sel] (the merge of its forward partials runs
    inside fwd[win] and the sum of its dQ partials inside dq[cmp+win]);
    window = fwd[win] + dkdv[win] (fwd[win] carries that merge and the gate
    blend); compression = fwd[cmp] + dkdv[cmp]; the combined dQ launch on its
    own.  `measure_branches` gives the per-branch split."""
    def frac(names, flop_names=None):
        names = [n for n in names if n in iso_spans]
        if not names:
            return None
        t = sum(iso_spans[n][1] for n in names) / ISO_STEPS / 1e3
        f = sum(flops_of[n] for n in (flop_names or names) if n in flops_of)
        return {"ms_per_step": round(t * 1e3, 4), "tflop": round(f / 1e12, 4),
                "mfma_frac": round(f / t / 1e12 / peak, 4) if t > 0 else None}
    return {
        "selection": frac(["fwd[sel]", "dkdv[sel]"]),
        "window": frac(["fwd[win]", "dkdv[win]"]),
        "compression": frac(["fwd[cmp]", "dkdv[cmp]"]),
        "range_dq": frac(["dq[cmp+win]"]),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-rows", type=int, default=1024,
                    help="query rows of the CPU baseline sample (about 10-20 s of CPU work at c3)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0: min(16, os.cpu_count())")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the forced-block variant and the c1 timings")
    ap.add_argument("--spans", action="store_true", help="print the per-call HIP-event breakdown to stderr")
    ap.add_argument("--no-branches", action="store_true",
                    help="skip the per-branch pass (its unfused launches would mix into a profile's per-kernel "
                         "statistics)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (3 times): the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda:0").random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy probe: 3 copies of {args.copy_probe_mib} MiB")
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the NSA layer shards over (B, Hkv) with no communication)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    name = args.workload
    w = WORKLOADS[name]
    if w["kind"] in ("model", "forward", "decode"):
        if w["kind"] == "decode":
            extra = run_decode_bench(w, steps=max(args.steps, 50), warmup=args.warmup)
        else:
            extra = run_model_bench(args, w) if w["kind"] == "model" else run_forward_bench(args, w, name)
        print(json.dumps({"workload": name, "desc": w["desc"], "steps": args.steps, "warmup": args.warmup,
                          "result": extra}), flush=True)
        return
    r = run_gpu(args, w, name)
    ms, spans, iso_spans, dom_name, flops_of, kv = r["ms"], r["spans"], r["iso_spans"], r["dom"], r["flops_of"], \
        r["kv"]
    tokens = w["B"] * w["T"]
    value = tokens / (ms / 1e3)
    total_flops = step_flops(w, kv)

    if args.spans:
        for nm, (calls, tot) in sorted(iso_spans.items(), key=lambda x: -x[1][1]):
            log(f"  {nm:28s} calls {calls:4d}  total {tot:9.3f} ms  per step {tot / ISO_STEPS:8.3f} ms")
    roofline = None
    if dom_name is not None and dom_name in spans:
        calls, tot = spans[dom_name]
        per_launch_s = tot / calls / 1e3
        roofline = roofline_of(w, dom_name, flops_of[dom_name], per_launch_s, MEASURED_TRAFFIC.get((name, dom_name)),
                               kv, r["pairs"])
        if dom_name in iso_spans:
            icalls, itot = iso_spans[dom_name]
            roofline["isolated_launch_ms"] = round(itot / icalls, 4)
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v with per-head scale U(0.5,2), gate logits N(0,1), dO N(0,1))",
        "config": {"workload": w["desc"], "B": w["B"], "T": w["T"], "Hq": w["Hq"], "Hkv": w["Hkv"], "D": w["D"],
                   "geometry": dict(zip(["cmp_block", "cmp_stride", "sel_block", "n_sel", "window", "force_init",
                                         "n_local"], w["geom"])),
                   "parallelism": "single GPU"},
        "mfu": round(total_flops / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "algorithmic_tflop_per_step": round(total_flops / 1e12, 3),
        "visible_keys": {"win": kv[0], "cmp": kv[1], "sel": kv[2]},
        "selection_pairs": r["pairs"],
        "roofline": roofline,
        "fwd_bwd_split": r["split"],
        "branches": (measure_branches(w, r["geom"], r["ins"], r["do"], kv)
                     if w["kind"] == "fused" and not args.no_branches else None),
        "fused_launches_by_branch": branch_fractions(iso_spans, flops_of, PEAK_BF16_TFLOPS),
        "per_kernel": per_kernel_table(iso_spans, flops_of, PEAK_BF16_TFLOPS, name),
        "memory": r["mem"],
    }
    if not args.no_extras and name == "c3":
        ms_f, kv_f = time_gpu_only(args, WORKLOADS["c3_forced"], "c3_forced")
        res["c3_forced"] = {"ms_per_step": round(ms_f, 3), "value": round(tokens / (ms_f / 1e3), 1),
                            "mfu": round(step_flops(WORKLOADS["c3_forced"], kv_f) / (ms_f / 1e3) / 1e12
                                         / PEAK_BF16_TFLOPS, 4)}
    if not args.no_extras and name == "c3":
        res["decode"] = {k: run_decode_bench(WORKLOADS[k]) for k in ("dec", "dec_b1")}
        res["phi"] = run_phi_bench()
        res.update(run_other_configs(args))
    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    if not args.no_cpu_baseline:
        log(f"[bench] CPU baseline: float32 oracle, {args.cpu_rows} rows, {threads} threads")
        tps, secs, nrows = run_cpu_baseline(w, r["ins"], r["do"], args.cpu_rows, threads) \
            if w["kind"] == "fused" else (None, None, None)
        if tps is not None:
            res["cpu_baseline"] = {
                "value": round(tps, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"{nrows} evenly spaced query rows of the same workload (fwd+bwd incl. importance/top-n "
                          f"for those rows), {secs:.1f} s, extrapolated linearly to tokens/s; CPU {cpu_model()}, "
                          f"os.cpu_count()={os.cpu_count()}"}
        if not args.no_extras:
            log("[bench] CPU baseline: config 1, dense float32 oracle")
            c1 = run_cpu_c1(threads)
            g1 = time_gpu_c1()
            res["cpu_baseline_c1"] = {
                v: {"cpu_tokens_per_s": round(tps1, 1), "cpu_ms": round(s1 * 1e3, 2), "gpu_f32_ms": round(g1[v], 3),
                    "gpu_f32_tokens_per_s": round(WORKLOADS["c1"]["T"] / (g1[v] / 1e3), 1)}
                for v, (tps1, s1) in c1.items()}
            res["cpu_baseline_c1"]["note"] = (f"B1 T1024 Hq4 Hkv1 D64 fwd+bwd float32, dense oracle, median of 3 "
                                              f"after 1 warm-up, {threads} threads; GPU: same inputs, float32")
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
