"""NSA fused forward + backward throughput on one MI355X.

A step is one full NSA attention layer call, forward and backward, over one
batch of synthetic inputs resident in HBM: compression pooling, compression
attention, block importance + top-n on the GPU, selection and sliding-window
attention, gate blend, then the backward of all of it.  The default workload
is BASELINE config 3 (B1 T32768 Hq64 Hkv4 D128, l=32 d=16 l'=64 top-16 with
the initial and two local blocks forced, w=512, bf16).

Prints ONE JSON line (rank 0): the metric, tokens/s, the dominant kernel's
roofline (algorithmic FLOPs / its HIP-event-timed launch duration) and a CPU
baseline (the float32 CPU oracle on a bounded sample of query rows).
"""

import argparse
import json
import os
import platform
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

WORKLOADS = {
    "c3": dict(B=1, T=32768, Hq=64, Hkv=4, D=128, geom=(32, 16, 64, 16, 512, True, 2), head_scale=True,
               desc="BASELINE config 3: fused 3-branch NSA fwd+bwd, B1 T32768 Hq64 Hkv4 D128, "
                    "l32/d16 l'64 top-16 (init + 2 local forced) w512, bf16"),
    "c2": dict(B=4, T=8192, Hq=16, Hkv=1, D=64, geom=(32, 16, 64, 16, 512, False, 0), head_scale=False,
               desc="BASELINE config 2 shape through the full NSA layer: B4 T8192 Hq16 Hkv1 D64"),
    "small": dict(B=1, T=4096, Hq=16, Hkv=1, D=128, geom=(32, 16, 64, 16, 512, True, 2), head_scale=True,
                  desc="reduced c3-like shape for quick checks"),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(w, dev, dtype, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    B, T, Hq, Hkv, D = w["B"], w["T"], w["Hq"], w["Hkv"], w["D"]

    def rn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32)

    q = rn(B, Hq, T, D)
    kv = [rn(B, Hkv, T, D) for _ in range(6)]
    if w["head_scale"]:
        sq = torch.rand(Hq, generator=g, device=dev) * 1.5 + 0.5
        skv = torch.rand(6, Hkv, generator=g, device=dev) * 1.5 + 0.5
        q = q * sq[None, :, None, None]
        kv = [x * skv[i][None, :, None, None] for i, x in enumerate(kv)]
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


def kernel_flops(w, kv):
    """Algorithmic FLOPs of one launch of each timed kernel (span name -> flops).

    Per (query head, visible key): forward 4*D (QK^T and PV); range dK/dV
    kernels 8*D (S, dP, dV, dK); range dQ kernels 2*D (dQ only: their S and
    dP are recomputed work, counted once in the dK/dV kernel).  The selection
    dK/dV kernel also forms the dQ partials (10*D); dq[sel] only sums them
    and has no FLOP model.  Sum = 14*D per key, the fwd+bwd convention of
    the metric.
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
    out["dq[cmp+win]"] = out["dq[cmp]"] + out["dq[win]"]   # both branches in one launch
    return out


# HBM bytes per launch of the dominant kernel, measured with two rocprofv3
# PMC passes of this bench (FETCH_SIZE, then WRITE_SIZE) and scaled by what
# the same counters read for a plain 1 GiB device copy (x2.0 and x1.0); the
# commands and counter values are kept under profiles/.  Reported only for
# the workload and kernel they were measured on.
ISO_STEPS = 2   # untimed steps with every call timed (per-kernel spans, dominant kernel)

MEASURED_TRAFFIC = {("c3", "dkdv[sel]"): 1.941e10 + 9.30e9}


def run_gpu(args, w):
    import nsa_fused_kernel as nfk
    import nsa_hip_ops as ops

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    geom = ops.NSAGeometry(*w["geom"])
    ins, do = make_inputs(w, dev, dtype)
    xs = [t.requires_grad_() for t in ins]

    def step():
        for x in xs:
            x.grad = None
        out, idx = nfk.nsa_attention(*xs, geom)
        out.backward(do)
        return idx

    log(f"[bench] warmup {args.warmup} step(s) on {torch.cuda.get_device_name(0)}")
    idx = None
    for _ in range(args.warmup):
        idx = step()
    torch.cuda.synchronize()
    if idx is None:
        idx = step()
        torch.cuda.synchronize()
    kv = keys_visible(w, idx)
    flops_of = kernel_flops(w, kv)
    # untimed, first: every call timed, with the backward's streams serialised
    # (nsa_hip_ops.OVERLAP_SEL_BWD off), so that each kernel's duration is its
    # own; this picks the dominant kernel
    iso = ops.LaunchTimer()
    overlap = ops.OVERLAP_SEL_BWD
    ops.OVERLAP_SEL_BWD = False
    try:
        ops.set_timer(iso)
        for _ in range(ISO_STEPS):
            step()
        torch.cuda.synchronize()
    finally:
        ops.set_timer(None)
        ops.OVERLAP_SEL_BWD = overlap
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
    return ms, timer.summary_ms(), iso_spans, dom, flops_of, kv, ins, do


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


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


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
    ap.add_argument("--spans", action="store_true", help="print the per-call HIP-event breakdown to stderr")
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
              "(the NSA layer shards over (B, Hkv) with no communication; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    w = WORKLOADS[args.workload]
    ms, spans, iso_spans, dom_name, flops_of, kv, ins_dev, do_dev = run_gpu(args, w)
    tokens = w["B"] * w["T"]
    value = tokens / (ms / 1e3)
    total_flops = sum(flops_of.values())

    # dominant kernel: the call with a FLOP model and the largest total time
    # in the untimed steps; its launches in the timed steps give `achieved`
    if args.spans:
        for name, (calls, tot) in sorted(iso_spans.items(), key=lambda x: -x[1][1]):
            log(f"  {name:28s} calls {calls:4d}  total {tot:9.3f} ms  per step {tot / ISO_STEPS:8.3f} ms")
    roofline = None
    if dom_name is not None and dom_name in spans:
        name = dom_name
        calls, tot = spans[name]
        per_launch_s = tot / calls / 1e3
        achieved = flops_of[name] / per_launch_s / 1e12
        roofline = {"bound": "mfma", "kernel": name, "achieved": round(achieved, 2),
                    "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                    "traffic": MEASURED_TRAFFIC.get((args.workload, name)),
                    "launch_ms": round(per_launch_s * 1e3, 4)}
        if name in iso_spans:
            # the same kernel in the untimed steps (backward serialised)
            icalls, itot = iso_spans[name]
            iso_s = itot / icalls / 1e3
            roofline["isolated"] = {"launch_ms": round(iso_s * 1e3, 4),
                                    "achieved": round(flops_of[name] / iso_s / 1e12, 2),
                                    "frac": round(flops_of[name] / iso_s / 1e12 / PEAK_BF16_TFLOPS, 4)}
    cpu = None
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        log(f"[bench] CPU baseline: float32 oracle, {args.cpu_rows} rows, {threads} threads")
        tps, secs, nrows = run_cpu_baseline(w, ins_dev, do_dev, args.cpu_rows, threads)
        cpu = {"value": round(tps, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
               "sample": f"{nrows} evenly spaced query rows of the same workload (fwd+bwd incl. importance/top-n "
                         f"for those rows), {secs:.1f} s, extrapolated linearly to tokens/s; CPU {cpu_model()}, "
                         f"os.cpu_count()={os.cpu_count()}"}
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
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
