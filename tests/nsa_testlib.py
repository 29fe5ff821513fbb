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


# Tolerances (north star): bf16 max-abs 2e-2 and rel-L2 1e-2, fp32 1e-4; the
# max-abs bound is relative to the reference's largest magnitude when that
# exceeds 1 (a bf16 value v carries a rounding error of up to |v| * 2^-9).
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
    atol, rtol = TOL[dtype]
    assert torch.isfinite(got.detach().float().cpu()).all(), f"{what}: non-finite values"
    max_abs, rel_l2, scale = errors(got, ref)
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


def assert_strict(got, ref, dtype, what=""):
    atol, ulp, rtol = STRICT[dtype]
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
