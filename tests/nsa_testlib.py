"""Shared helpers of the parity tests: seeded inputs, tolerances, configs.

Inputs are drawn on the CPU from a torch.Generator, rounded to the test dtype
and then copied to the GPU, so the float64 oracle sees exactly the values the
kernels see.
"""

import math

import torch

# The reference kernel-test matrix (test_kernel.py:25-33): G in {1,2,3,4}, D in
# {32,64,128}, block in {16,32,64}, S up to 32 (more than some rows' valid blocks).
REF_CONFIGS = [
    dict(B=2, Hq=4, Hkv=2, D=32, T=256, block_size=16, S=4),
    dict(B=1, Hq=8, Hkv=2, D=64, T=512, block_size=32, S=8),
    dict(B=2, Hq=12, Hkv=4, D=64, T=512, block_size=16, S=8),
    dict(B=1, Hq=16, Hkv=4, D=128, T=1024, block_size=64, S=16),
    dict(B=1, Hq=4, Hkv=4, D=64, T=384, block_size=16, S=6),
    dict(B=2, Hq=6, Hkv=3, D=32, T=256, block_size=32, S=3),
    dict(B=1, Hq=8, Hkv=2, D=64, T=512, block_size=16, S=32),
]

# GQA-16 cases shaped like the BASELINE configs (reduced T), plus G > 16 and D = 16.
G16_CONFIGS = [
    dict(B=1, Hq=32, Hkv=2, D=128, T=1024, block_size=64, S=16),
    dict(B=2, Hq=16, Hkv=1, D=64, T=768, block_size=64, S=16),
    dict(B=1, Hq=40, Hkv=2, D=64, T=320, block_size=32, S=5),
    dict(B=1, Hq=4, Hkv=2, D=16, T=200, block_size=16, S=4),
]


def cfg_id(c):
    return "B{B}-Hq{Hq}-Hkv{Hkv}-D{D}-T{T}-bs{block_size}-S{S}".format(**c)


def window_for(c):
    """Not a multiple of the block or the kernel tile (test_kernel_fused.py:29-31)."""
    return min(c["T"], 2 * c["block_size"] + 5)


def randn(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def make_block_idx(B, Hkv, T, block_size, S, seed=0):
    """Random causal, duplicate-free block lists with -1 padding
    (the reference's generator, test_kernel.py:39-58)."""
    g = torch.Generator().manual_seed(seed)
    n_blk = T // block_size
    valid = (torch.arange(n_blk)[None, :] + 1) * block_size <= (torch.arange(T)[:, None] + 1)
    score = torch.rand(B, Hkv, T, n_blk, generator=g).masked_fill(~valid[None, None], -1.0)
    k = min(S, n_blk)
    topv, topi = score.topk(k, dim=-1)
    sel = torch.where(topv >= 0, topi.to(torch.int32), torch.full_like(topi, -1, dtype=torch.int32))
    idx = torch.full((B, Hkv, T, S), -1, dtype=torch.int32)
    idx[..., :k] = sel
    return idx


# Tolerances (north star): bf16 max-abs 2e-2 and rel-L2 1e-2, fp32 1e-4.
TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float32: (1e-4, 1e-5)}


def errors(got, ref):
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    diff = (g - r)
    max_abs = float(diff.abs().max()) if diff.numel() else 0.0
    denom = float(r.norm())
    rel_l2 = float(diff.norm()) / denom if denom > 0 else float(diff.norm())
    scale = max(1.0, float(r.abs().max()) if r.numel() else 1.0)
    return max_abs, rel_l2, scale


def assert_close(got, ref, dtype, what=""):
    """The reduced-shape gate: max-abs atol relative to the reference's
    largest magnitude when that exceeds 1, and rel-L2 <= rtol.  These tests
    use unit-variance inputs without the 1/sqrt(D) damping, as the
    reference's own kernel tests do (test_kernel_backward.py:35-39): rows are
    peaked and gradients reach |g| ~ 100 (the pooled token every query sees).
    With bf16 P / dS operands (the FlashAttention convention) a gradient's
    error scales with the sum of the magnitudes of its terms, not with the
    element, so it is bounded against the tensor's scale; the BASELINE-shape
    checks use the elementwise ``assert_strict`` and ``assert_letter``."""
    atol, rtol = TOL[dtype]
    assert torch.isfinite(got.detach().float().cpu()).all(), f"{what}: non-finite values"
    max_abs, rel_l2, scale = errors(got, ref)
    log(f"  {what:12s} max_abs {max_abs:.3e}  rel_l2 {rel_l2:.3e}  |ref|max {scale:.3e}")
    assert max_abs <= atol * scale, f"{what}: max_abs {max_abs:.3e} > {atol:.1e} * {scale:.2f}"
    assert rel_l2 <= rtol, f"{what}: rel_l2 {rel_l2:.3e} > {rtol:.1e}"
    return max_abs, rel_l2


def to64(*ts):
    return [t.detach().double().cpu().clone() for t in ts]


def require_gpu():
    import pytest
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def log(msg):
    print(msg, flush=True)


__all__ = ["REF_CONFIGS", "G16_CONFIGS", "cfg_id", "window_for", "randn", "make_block_idx", "TOL",
           "errors", "assert_close", "to64", "require_gpu", "log", "math"]


# Strict form of the north-star bound for the full-shape BASELINE checks:
# elementwise |got - ref| <= atol + ulp * |ref| (atol the north star's
# absolute bound; ulp one storage unit of the dtype at the value's own
# magnitude, the representation limit of a bf16 output: 2^-8), and
# rel-L2 <= rtol.  No scaling by the tensor's largest value.
STRICT = {torch.bfloat16: (2e-2, 2.0 ** -8, 1e-2), torch.float32: (1e-4, 0.0, 1e-5)}


def assert_strict(got, ref, dtype, what="", ulp=None):
    atol, ulp0, rtol = STRICT[dtype]
    ulp = ulp0 if ulp is None else ulp
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, f"{what}: shape {tuple(g.shape)} vs {tuple(r.shape)}"
    assert torch.isfinite(g).all(), f"{what}: non-finite values"
    diff = (g - r).abs()
    max_abs = float(diff.max()) if diff.numel() else 0.0
    denom = float(r.norm())
    rel_l2 = float((g - r).norm()) / denom if denom > 0 else float((g - r).norm())
    excess = float((diff - (atol + ulp * r.abs())).max()) if diff.numel() else -1.0
    ref_max = float(r.abs().max()) if r.numel() else 0.0
    log(f"  {what:12s} max_abs {max_abs:.3e}  rel_l2 {rel_l2:.3e}  |ref|max {ref_max:.3e}")
    assert excess <= 0.0, f"{what}: max_abs {max_abs:.3e} exceeds {atol:.0e} + {ulp:.1e}|ref| (by {excess:.3e})"
    assert rel_l2 <= rtol, f"{what}: rel_l2 {rel_l2:.3e} > {rtol:.1e}"
    return max_abs, rel_l2


__all__ += ["STRICT", "assert_strict"]


def bf16_units(got, ref):
    """|got - ref| in units of the bf16 spacing at |ref| (2^(e - 7) for
    |ref| in [2^e, 2^(e+1)))."""
    r = ref.detach().double().cpu()
    e = torch.floor(torch.log2(r.abs().clamp(min=2.0 ** -126)))
    return (got.detach().double().cpu() - r).abs() / torch.pow(2.0, e - 7)


def assert_letter(got, ref, what="", got32=None, failures=None):
    """The north star's bound taken literally: max |value - ref| <= 2e-2 and
    rel-L2 <= 1e-2 against the float64 reference, where `value` is what the
    kernels computed before the output's final bf16 rounding (``got32``: the
    same launches with a float32 destination), and the bf16 output ``got`` is
    exactly the round-to-nearest-even of that value.  Without ``got32`` the
    bf16 output itself must meet the bound.  Also logged: the bf16 output
    against the bf16-rounded reference (max-abs; the largest distance in
    bf16 units where |ref| >= 1; how many elements are over 2e-2 and the
    smallest |ref| among them: a bf16 unit is 2^-5 at |ref| in [4, 8) and
    2^-4 in [8, 16), so a value within 2e-2 may round to a neighbour of
    bf16(ref) that is more than 2e-2 away).  With ``failures`` (a list) a
    miss is appended to it instead of raised."""
    r = ref.detach().double().cpu()
    if got32 is not None:
        assert got32.dtype == torch.float32, f"{what}: the unrounded value must be float32"
        same = torch.equal(got.detach().cpu(), got32.detach().cpu().to(got.dtype))
        assert same, f"{what}: the bf16 output is not the rounding of the float32 value"
        v = got32.detach().double().cpu()
    else:
        v = got.detach().double().cpu()
    d = (v - r).abs()
    max_abs = float(d.max()) if d.numel() else 0.0
    denom = float(r.norm())
    rel_l2 = float((v - r).norm()) / denom if denom > 0 else float((v - r).norm())
    rb = r.to(torch.bfloat16)
    gb = got.detach().cpu()
    db = (gb.double() - rb.double()).abs()
    big = r.abs() >= 1.0
    units = float(bf16_units(gb[big], rb.double()[big]).max()) if int(big.sum()) else 0.0
    over = db > 2e-2
    n_over = int(over.sum())
    min_ref_over = float(r.abs()[over].min()) if n_over else float("nan")
    log(f"  {what:12s} letter: max|value - ref| {max_abs:.3e}  rel_l2 {rel_l2:.3e}"
        f"{' (float32 value; bf16 output = its rounding)' if got32 is not None else ' (bf16 output)'};"
        f"  bf16 output vs bf16(ref): max_abs {float(db.max()):.3e}, max {units:.0f} unit(s) at |ref| >= 1, "
        f"{n_over} element(s) over 2e-2 (smallest |ref| among them {min_ref_over:.2f})")
    msgs = []
    if max_abs > 2e-2:
        msgs.append(f"{what}: max |value - ref| {max_abs:.3e} > 2e-2")
    if rel_l2 > 1e-2:
        msgs.append(f"{what}: rel_l2 {rel_l2:.3e} > 1e-2")
    if msgs and failures is None:
        raise AssertionError("; ".join(msgs))
    if failures is not None:
        failures.extend(msgs)
    return max_abs, rel_l2


__all__ += ["bf16_units", "assert_letter"]
