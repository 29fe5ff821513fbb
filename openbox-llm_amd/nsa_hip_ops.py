"""Host side of the MI355X NSA path: tensor plumbing around libnsa_hip.so.

Every function here allocates its outputs with torch on the inputs' device and
launches HIP kernels on the current stream through the C-ABI (``_nsa_lib``).
Nothing falls back to another implementation: the library must load.

Branch semantics follow the reference (paths relative to its checkout):
selection nsa_selection_kernel.py:55-92, window / compression
nsa_fused_kernel.py:576-597, importance / top-n nsa_model.py:245-258, gate
nsa_fused_kernel.py:572-573.  The compression geometry is generalised to a
span ``cmp_block`` with stride ``cmp_stride`` (the reference is the aligned
case ``cmp_block == cmp_stride == block_size``).
"""

from __future__ import annotations

import contextlib
from collections import defaultdict
from dataclasses import dataclass

import torch

import _nsa_lib as L

MODE_WINDOW = L.MODE_WINDOW
MODE_COMPRESS = L.MODE_COMPRESS
SEL_DKDV_CHUNK = 512          # CSR queries per selection dK/dV work item (deterministic partials: 512 measured
                              # 0.1 ms a c3 step and 0.09 ms a c4 layer faster than 1024)
SEL_FWD_CHUNK = 128           # CSR queries per selection forward work item (c3: 128 measured 0.1 ms faster than 512)


@dataclass(frozen=True)
class NSAGeometry:
    """Block geometry of one NSA layer.

    cmp_block / cmp_stride: compression span l and stride d; sel_block: l';
    n_sel: top-n count (forced blocks included); window: w; force_init and
    n_local force block 0 and the n_local most recent blocks into the top-n.
    ``NSAGeometry.aligned(bs, n, w)`` is the reference grid
    (nsa_model.py:134-140): l = d = l' = bs, no forcing.
    """

    cmp_block: int
    cmp_stride: int
    sel_block: int
    n_sel: int
    window: int
    force_init: bool = False
    n_local: int = 0

    @staticmethod
    def aligned(block_size, n_sel, window):
        return NSAGeometry(block_size, block_size, block_size, n_sel, window)


# ---------------------------------------------------------------------------
# optional per-launch timing (HIP events on the launching stream)
# ---------------------------------------------------------------------------

class LaunchTimer:
    """Collects (start, end) HIP events around every library call, by name.

    Installed with ``set_timer``; the events are recorded on the current
    stream, which is the stream every kernel of the call is launched on.
    ``only``: the call names to time (None: all).  Every timing event is a
    packet in the stream's queue, so a timer meant to leave the timed work
    undisturbed records only the calls it reports.
    """

    def __init__(self, only=None):
        self.spans = defaultdict(list)
        self.only = None if only is None else frozenset(only)

    def wants(self, name):
        return self.only is None or name in self.only

    @contextlib.contextmanager
    def span(self, name):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        try:
            yield
        finally:
            b.record()
            self.spans[name].append((a, b))

    def summary_ms(self):
        """name -> (calls, total ms); call after a device synchronize."""
        return {k: (len(v), sum(a.elapsed_time(b) for a, b in v)) for k, v in self.spans.items()}


_TIMER = None


def set_timer(timer):
    global _TIMER
    _TIMER = timer


def _span(name):
    return _TIMER.span(name) if _TIMER is not None and _TIMER.wants(name) else contextlib.nullcontext()


def _span_name(kind, mode):
    return f"{kind}[{'win' if mode == MODE_WINDOW else 'cmp'}]"


def _call(name, fn, *args):
    with _span(name):
        rc = fn(*args)
    L.check(rc, name)


# ---------------------------------------------------------------------------
# argument checks (the reference's asserts, nsa_selection_kernel.py:186-189)
# ---------------------------------------------------------------------------

def _contig(x):
    """Dense row-major with a 16-byte aligned base (the kernels read 16-byte rows)."""
    if not x.is_contiguous():
        x = x.contiguous()
    if x.data_ptr() % 16 != 0:
        x = x.clone()
    return x


def check_qkv(q, k, v=None):
    assert q.dim() == 4 and k.dim() == 4, "q/k/v must be [B, H, T, D]"
    assert q.is_cuda and k.is_cuda, "NSA HIP kernels need GPU tensors"
    B, Hq, T, D = q.shape
    assert k.shape[0] == B and k.shape[3] == D, "q/k batch or head dim mismatch"
    assert Hq % k.shape[1] == 0, "GQA needs n_q_heads divisible by n_kv_heads"
    assert D in (16, 32, 64, 128), "head dim must be a power of two <= 128"
    assert q.stride(-1) == 1 and k.stride(-1) == 1, "head dim must be contiguous"
    assert k.dtype == q.dtype, "q/k dtype mismatch"
    if v is not None:
        assert v.shape == k.shape and v.dtype == q.dtype and v.stride(-1) == 1
    L.dtype_code(q)


def _lib():
    return L.load()


def _stream(t):
    return L.stream_of(t)


_SIDE_STREAMS = {}

# True: the fused backward runs the selection dK/dV on a side stream, beside
# the window and compression key-side kernels.  False (default): everything
# runs in order on the current stream.  At c3 on MI355X the overlap is slower:
# 22.9-23.0 against 22.3 ms per fwd+bwd step, and 23.2 ms with the selection
# dK/dV's persistent grid halved to one workgroup per CU to leave room beside
# it (alone, that grid takes 7.5 instead of 5.0 ms: the kernel needs both
# workgroups per CU for its memory traffic).  In order, each kernel's timing
# describes that kernel alone.
OVERLAP_SEL_BWD = False

# True: the fused backward computes the compression and window dQ in one launch
# (nsa_range_dq_cw) that also finishes the rows; False: one launch per branch
# through a float32 dQ buffer (the compression dQ finishing the rows, or, with
# SEPARATE_SEL_DQ, a third launch summing the selection partials), so that
# each branch's dQ can be timed on its own.
FUSE_RANGE_DQ = True
SEPARATE_SEL_DQ = False


def _side_stream(device):
    """A second stream per device (default priority) for work that overlaps the
    current stream's."""
    key = torch.device(device).index
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
    return _SIDE_STREAMS[key]


def padded_len(n):
    return int(_lib().nsa_padded_len(int(n)))


# ---------------------------------------------------------------------------
# layout helpers
# ---------------------------------------------------------------------------

def transpose_kv(x):
    """[B,H,Lk,D] -> [B,H,D,padded_len(Lk)] key-contiguous copy (zero pad)."""
    x = _contig(x)
    B, H, Lk, D = x.shape
    Lp = padded_len(Lk)
    xt = torch.empty(B, H, D, Lp, device=x.device, dtype=x.dtype)
    _call("nsa_transpose_kv", _lib().nsa_transpose_kv, L.ptr(x), L.ptr(xt), B * H, Lk, D, Lp, L.dtype_code(x),
                                    _stream(x))
    return xt


def pack_heads(x, Hkv):
    """[B,Hkv*G,T,D] -> [B,Hkv,T,G,D]: the G heads of one query and KV head
    contiguous, the query-side layout of the selection kernels."""
    x = _contig(x)
    B, Hq, T, D = x.shape
    assert Hq % Hkv == 0, "query heads must be a multiple of the KV heads"
    G = Hq // Hkv
    xp = torch.empty(B, Hkv, T, G, D, device=x.device, dtype=x.dtype)
    _call("nsa_pack_heads", _lib().nsa_pack_heads, L.ptr(x), L.ptr(xp), B, Hkv, G, T, D, L.dtype_code(x),
          _stream(x))
    return xp


def cast_f32(x, dtype):
    if dtype == torch.float32:
        return x
    y = torch.empty(x.shape, device=x.device, dtype=dtype)
    code = L.NSA_BF16 if dtype == torch.bfloat16 else None
    assert code is not None, f"dtype {dtype} is not supported"
    _call("nsa_cast_f32", _lib().nsa_cast_f32, L.ptr(x), L.ptr(y), x.numel(), code, _stream(x))
    return y


# ---------------------------------------------------------------------------
# pooling
# ---------------------------------------------------------------------------

def n_cmp_tokens(T, l, d):
    return (T - l) // d + 1 if T >= l else 0


def pool_fwd(x, l, d):
    x = _contig(x)
    B, H, T, D = x.shape
    n = n_cmp_tokens(T, l, d)
    out = torch.empty(B, H, n, D, device=x.device, dtype=x.dtype)
    if n > 0:
        _call("nsa_pool_fwd", _lib().nsa_pool_fwd, L.ptr(x), L.ptr(out), B, H, T, D, l, d, L.dtype_code(x),
                                    _stream(x))
    return out


def pool_bwd(dpool, T, l, d, dtype):
    dpool = _contig(dpool)
    B, H, n, D = dpool.shape
    dx = torch.empty(B, H, T, D, device=dpool.device, dtype=dtype)
    if T > 0:
        _call("nsa_pool_bwd", _lib().nsa_pool_bwd, L.ptr(dpool), L.dtype_code(dpool), L.ptr(dx), B, H, T, D, l, d,
                                    L.NSA_F32 if dtype == torch.float32 else L.NSA_BF16,
                                    _stream(dpool))
    return dx


class WeightedPoolHIP(torch.autograd.Function):
    """``out[b,h,i] = sum_p w[p] (x[b,h,i d + p] + pos[p])`` (float32
    ``[B,H,n,D]``): the pooling of BlockCompressor (nsa_model.py:100-123,
    before its projection) on the HIP kernels, over the overlapping spans in
    place.  Gradients for x (in x's dtype), w and pos (float32 sums)."""

    @staticmethod
    def forward(ctx, x, w, pos, l, d):
        x = _contig(x)
        B, H, T, D = x.shape
        assert w.shape == (l,) and pos.shape == (l, D), "weighted pool: w [l], pos [l, D]"
        n = n_cmp_tokens(T, l, d)
        with torch.autocast("cuda", enabled=False):
            wf = w.float().contiguous()
            cvec = (wf @ pos.float()).contiguous()
        out = torch.empty(B, H, n, D, device=x.device, dtype=torch.float32)
        if n > 0:
            _call("nsa_wpool_fwd", _lib().nsa_wpool_fwd, L.ptr(x), L.ptr(wf), L.ptr(cvec), L.ptr(out), B, H, T, D,
                  l, d, L.dtype_code(x), _stream(x))
        ctx.save_for_backward(x, wf, pos)
        ctx.meta = (l, d, w.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, wf, pos = ctx.saved_tensors
        l, d, w_dtype = ctx.meta
        B, H, T, D = x.shape
        dout = _contig(dout.float())
        dx = torch.empty_like(x)
        dw_part = torch.empty(l, B * H, device=x.device, dtype=torch.float32)
        _call("nsa_wpool_bwd", _lib().nsa_wpool_bwd, L.ptr(dout), L.ptr(wf), L.ptr(dx), B, H, T, D, l, d,
              L.dtype_code(x), _stream(x))
        _call("nsa_wpool_dw", _lib().nsa_wpool_dw, L.ptr(x), L.ptr(dout), L.ptr(dw_part), B, H, T, D, l, d,
              L.dtype_code(x), _stream(x))
        with torch.autocast("cuda", enabled=False):
            dc = dout.sum(dim=(0, 1, 2))                  # the gradient of cvec = w^T pos
            dw = dw_part.sum(dim=1) + pos.float() @ dc
            dpos = wf[:, None] * dc[None, :]
        return dx, dw.to(w_dtype), dpos.to(pos.dtype), None, None


def weighted_pool(x, w, pos, l, d):
    """BlockCompressor's pooled tokens before the projection, ``sum_p w[p]
    (x[i d + p] + pos[p])`` for the spans [i d, i d + l) of ``x [B,H,T,D]``."""
    return WeightedPoolHIP.apply(x, w, pos, l, d)


def _seg_table(segs, bufs):
    """ctypes arrays (kept alive by the caller) for a segment table."""
    import ctypes
    n = len(segs)
    ints = ctypes.c_int * n
    heads = ints(*[int(s[0]) for s in segs])
    dims = ints(*[int(s[1]) for s in segs])
    rot = ints(*[1 if s[2] else 0 for s in segs])
    ptrs = (ctypes.c_void_p * n)(*[None if b is None else b.data_ptr() for b in bufs])
    return heads, dims, rot, ptrs


def _addr(arr):
    import ctypes
    return None if arr is None else ctypes.cast(arr, ctypes.c_void_p)


class HeadSplitHIP(torch.autograd.Function):
    """The stacked projection ``y [B,T,W]`` split into head-major tensors
    ``[B,H_k,T,hd_k]``, one per segment ``(H_k, hd_k, rotate_k)`` from column
    0 (columns past the segments are padding: ignored, zero gradient), in one
    kernel: the model's ``_split_heads(proj(x)).contiguous()`` per branch
    (nsa_model.py:192-194, 325-335), with the rotary embedding of a RoPE model
    (half-split pairs, factors ``cos``/``sin`` [T, hd/2] float32) and one
    segment's bias folded in.  The backward scatters the outputs' gradients
    back into the stacked row (inverse rotation) in one kernel."""

    @staticmethod
    def forward(ctx, y, bias, cos, sin, segs, bias_seg):
        y = _contig(y)
        B, T, W = y.shape
        assert len(segs) <= 8 and sum(h * d for h, d, _ in segs) <= W, "segments must fit the stacked row"
        rot = any(s[2] for s in segs)
        if rot:
            hd = {s[1] for s in segs if s[2]}
            assert len(hd) == 1 and cos is not None and sin is not None, "rotated segments share one head dim"
            assert cos.shape == (T, next(iter(hd)) // 2) and sin.shape == cos.shape, "rotary tables [T, hd/2]"
            cos = _contig(cos.float())
            sin = _contig(sin.float())
        outs = [torch.empty(B, h, T, d, device=y.device, dtype=y.dtype) for h, d, _ in segs]
        biases = None
        bf = None
        if bias is not None:
            H, d, _ = segs[bias_seg]
            assert bias.numel() == H * d, "the bias covers its segment"
            with torch.autocast("cuda", enabled=False):
                bf = bias.detach().float().contiguous()
            biases = [None] * len(segs)
            biases[bias_seg] = bf
        heads, dims, rots, ptrs = _seg_table(segs, outs)
        bptrs = None if biases is None else _seg_table(segs, biases)[3]
        _call("nsa_heads_split", _lib().nsa_heads_split, L.ptr(y), _addr(ptrs), _addr(bptrs), _addr(heads),
              _addr(dims), _addr(rots), len(segs), L.ptr(cos) if rot else None, L.ptr(sin) if rot else None, B, T, W,
              L.dtype_code(y), _stream(y))
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(cos if rot else None, sin if rot else None)
        ctx.meta = (segs, bias_seg, B, T, W, y.dtype, None if bias is None else bias.dtype)
        return tuple(outs)

    @staticmethod
    def backward(ctx, *gouts):
        cos, sin = ctx.saved_tensors
        segs, bias_seg, B, T, W, dtype, bias_dtype = ctx.meta
        gs = [None if g is None else _contig(g.to(dtype)) for g in gouts]
        dy = torch.empty(B, T, W, device=next(g for g in gs if g is not None).device, dtype=dtype) \
            if any(g is not None for g in gs) else None
        if dy is None:
            return (None,) * 6
        heads, dims, rots, ptrs = _seg_table(segs, gs)
        _call("nsa_heads_merge_grad", _lib().nsa_heads_merge_grad, _addr(ptrs), L.ptr(dy), _addr(heads),
              _addr(dims), _addr(rots), len(segs), L.ptr(cos), L.ptr(sin), B, T, W, L.dtype_code(dy), _stream(dy))
        dbias = None
        if bias_dtype is not None and ctx.needs_input_grad[1]:
            # float32 sums over B and T of the segment's gradient; the bias is
            # added before the rotation, so a rotated segment's gradient is
            # rotated back first (per t, after the sum over B)
            H, d, rot = segs[bias_seg]
            g = gouts[bias_seg]
            with torch.autocast("cuda", enabled=False):
                if g is None:
                    dbias = torch.zeros(H * d, device=dy.device, dtype=torch.float32)
                elif not rot:
                    dbias = g.float().sum(dim=(0, 2)).reshape(-1)       # [H, d] summed over B and T
                else:
                    gs = g.float().sum(dim=0)                           # [H, T, d]
                    h = d // 2
                    a, b = gs[..., :h], gs[..., h:]
                    gs = torch.cat([a * cos + b * sin, b * cos - a * sin], dim=-1)
                    dbias = gs.sum(dim=1).reshape(-1)
            dbias = dbias.to(bias_dtype)
        return dy, dbias, None, None, None, None


def split_heads(y, segs, cos=None, sin=None, bias=None, bias_seg=None):
    """Head-major tensors of the stacked projection ``y [B,T,W]`` per segment
    ``(heads, head_dim, rotate)``, rotated segments by the rotary factors
    ``cos``/``sin`` [T, head_dim/2], ``bias`` added to segment ``bias_seg``."""
    assert y.is_cuda, "the head split runs on the GPU"
    return HeadSplitHIP.apply(y, bias, cos, sin, tuple(tuple(s) for s in segs), bias_seg)


class _PoolMean(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, l, d):
        ctx.meta = (x.shape[2], l, d, x.dtype)
        return pool_fwd(x, l, d)

    @staticmethod
    def backward(ctx, dp):
        T, l, d, dtype = ctx.meta
        return pool_bwd(dp, T, l, d, dtype), None, None


def pool_mean(x, l, d):
    """Differentiable mean pool over spans [i*d, i*d+l)."""
    assert x.is_cuda and x.dim() == 4
    return _PoolMean.apply(x, l, d)


# ---------------------------------------------------------------------------
# forward kernels
# ---------------------------------------------------------------------------

def sel_fwd(q, k, v, block_idx, block_size, vt=None):
    """Selection forward -> (o, lse[f32])."""
    check_qkv(q, k, v)
    q, k = _contig(q), _contig(k)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    assert k.shape[2] == T, "selection keys must have the query length"
    assert block_idx.shape[:3] == (B, Hkv, T), "block_idx must be [B, Hkv, T, S]"
    assert block_size >= 16 and block_size % 16 == 0, "block_size must be a multiple of 16"
    idx = block_idx.to(torch.int32).contiguous()
    S = idx.shape[-1]
    if vt is None:
        vt = transpose_kv(v)
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, T, device=q.device, dtype=torch.float32)
    _call("fwd[sel]", _lib().nsa_sel_fwd, L.ptr(q), L.ptr(k), L.ptr(vt), L.ptr(idx), L.ptr(o), L.ptr(lse),
                               B, Hq, Hkv, T, D, S, block_size, L.dtype_code(q), _stream(q))
    return o, lse


def f16s_empty(shape, device):
    """A branch-output buffer in the library's NSA_F16S form: fp16 rows, each
    stored divided by a power-of-two scale (1 unless the row's largest
    magnitude reaches 2^15), followed in the same storage by the float32
    scales, one per row.  Returns the float16 view of the rows; only the
    library's kernels read it (``_nsa_lib.dtype_code`` checks the room for
    the scales)."""
    rows = shape[0] * shape[1] * shape[2]
    buf = torch.empty(rows * shape[3] + 2 * rows, device=device, dtype=torch.float16)
    return buf[:rows * shape[3]].view(shape)


def kept_output(shape, like):
    """The buffer of a branch output kept for the backward's row dots
    dO . o: NSA_F16S for 16-bit inputs (eight times finer than bf16, half of
    float32's bytes), float32 for float32 inputs."""
    if like.dtype == torch.float32:
        return torch.empty(shape, device=like.device, dtype=torch.float32)
    return f16s_empty(shape, like.device)


def range_fwd(mode, q, k, v, window=0, cmp_block=1, cmp_stride=1, vt=None, q_packed=None, o_f32=False,
              o_kept=False):
    """Window (mode 0) or compression (mode 1) forward -> (o, lse[f32]);
    ``q_packed`` (optional, [B, Hkv, T, G, D]) also receives the
    ``pack_heads`` copy of q.  ``o_f32``: o in float32 (unrounded);
    ``o_kept``: o in the form the fused layer keeps for its backward
    (``kept_output``); else o is in q's dtype."""
    check_qkv(q, k, v)
    q, k = _contig(q), _contig(k)
    B, Hq, T, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    if mode == MODE_WINDOW:
        assert Lk == T and window >= 1, "window keys must have the query length, window >= 1"
    if vt is None:
        vt = transpose_kv(v)
    if o_kept:
        o = kept_output(q.shape, q)
    else:
        o = torch.empty(q.shape, device=q.device, dtype=torch.float32 if o_f32 else q.dtype)
    lse = torch.empty(B, Hq, T, device=q.device, dtype=torch.float32)
    _call(_span_name("fwd", mode), _lib().nsa_range_fwd, mode, L.ptr(q), L.ptr(k), L.ptr(vt), L.ptr(o), L.ptr(lse),
          B, Hq, Hkv, T, Lk, D, int(window), int(cmp_block), int(cmp_stride), L.ptr(q_packed), L.dtype_code(q),
          L.dtype_code(o), _stream(q))
    return o, lse


def range_fwd_finish(q, k, v, window, sel_parts, idx, sel_block, o_c, gate, vt=None, out_f32=False):
    """Window forward that also finishes the gated layer's rows: returns
    (o_w, lse_w, o_s, lse_s, out), with the selection partials ``sel_parts``
    = (o_part, ml_part) of ``sel_fwd_partials`` merged into o_s / lse_s and
    out = sum_c sigmoid(gate_c) o_c over the three branches.  o_w and o_s
    take o_c's form (q's dtype, float32 unrounded, or the NSA_F16S form of
    ``kept_output``); out is in q's dtype, or float32 (unrounded) with
    ``out_f32``."""
    o_part, ml_part = sel_parts
    D = q.shape[-1]
    _check_sel_partials(o_part, q, _partial_dtype(q.dtype), "o_part", S=idx.shape[-1], block_size=sel_block)
    if ml_part.dtype != torch.float32 or ml_part.numel() * D != 2 * o_part.numel() or not ml_part.is_contiguous():
        raise TypeError("ml_part must hold one float32 (m, l) pair per partial row")
    check_qkv(q, k, v)
    q, k, gate, o_c = _contig(q), _contig(k), _contig(gate), _contig(o_c)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    assert gate.shape == (B, Hq, T, 3) and gate.dtype == q.dtype, "gate logits must be [B, Hq, T, 3] in q's dtype"
    if vt is None:
        vt = transpose_kv(v)
    assert o_c.dtype in (q.dtype, torch.float32, torch.float16), "branch outputs are q's dtype, float32 or NSA_F16S"
    if o_c.dtype == torch.float16:
        o_w, o_s = f16s_empty(q.shape, q.device), f16s_empty(q.shape, q.device)
    else:
        o_w = torch.empty(q.shape, device=q.device, dtype=o_c.dtype)
        o_s = torch.empty_like(o_w)
    lse_w = torch.empty(B, Hq, T, device=q.device, dtype=torch.float32)
    lse_s = torch.empty_like(lse_w)
    out = torch.empty(q.shape, device=q.device, dtype=torch.float32 if out_f32 else q.dtype)
    _call("fwd[win]", _lib().nsa_range_fwd_finish, MODE_WINDOW, L.ptr(q), L.ptr(k), L.ptr(vt), L.ptr(o_w),
          L.ptr(lse_w), B, Hq, Hkv, T, T, D, int(window), 1, 1, L.ptr(o_part), L.ptr(ml_part), L.ptr(idx),
          idx.shape[-1], int(sel_block), L.ptr(o_s), L.ptr(lse_s), L.ptr(o_c), L.ptr(gate), L.ptr(out),
          L.dtype_code(q), L.dtype_code(o_c), L.dtype_code(out), _stream(q))
    return o_w, lse_w, o_s, lse_s, out


def gate_fwd(gate, o_c, o_s, o_w):
    gate, o_c, o_s, o_w = (_contig(t) for t in (gate, o_c, o_s, o_w))
    assert gate.shape == o_c.shape[:3] + (3,), "gate logits must be [B, Hq, T, 3]"
    assert gate.dtype == o_c.dtype, "gate logits dtype must match q"
    out = torch.empty_like(o_c)
    rows = o_c.shape[0] * o_c.shape[1] * o_c.shape[2]
    _call("nsa_gate_fwd", _lib().nsa_gate_fwd, L.ptr(gate), L.ptr(o_c), L.ptr(o_s), L.ptr(o_w), L.ptr(out), rows,
                                o_c.shape[3], L.dtype_code(o_c), _stream(o_c))
    return out


def importance_topn(q, k_cmp, lse_cmp, geom: NSAGeometry, T=None, return_scores=False):
    """Block importance from the compression probabilities + top-n -> block_idx int32."""
    q, k_cmp = _contig(q), _contig(k_cmp)
    B, Hq, Tq, D = q.shape
    Hkv, n_cmp = k_cmp.shape[1], k_cmp.shape[2]
    T = Tq if T is None else T
    n_slc = T // geom.sel_block
    S = min(geom.n_sel, n_slc)
    idx = torch.empty(B, Hkv, T, S, device=q.device, dtype=torch.int32)
    scores = (torch.empty(B, Hkv, T, n_slc, device=q.device, dtype=torch.float32)
              if return_scores else None)
    if n_slc > 0:
        _call("nsa_importance_topn", _lib().nsa_importance_topn, 
            L.ptr(q), L.ptr(k_cmp), L.ptr(lse_cmp), L.ptr(idx), L.ptr(scores), B, Hq, Hkv, T, n_cmp, D,
            geom.cmp_block, geom.cmp_stride, geom.sel_block, geom.n_sel, int(geom.force_init),
            geom.n_local, L.dtype_code(q), _stream(q))
    return (idx, scores) if return_scores else idx


# ---------------------------------------------------------------------------
# backward kernels
# ---------------------------------------------------------------------------

def delta_of(do, o, lse, pack_hkv=0):
    """-> (dot, coff): dot[r] = dO[r] . O[r] in float32
    (nsa_selection_backward.py:168) and the row offset lse[r] * log2(e) that
    the dK/dV kernels take, both [B, Hq, T].  With ``pack_hkv`` > 0 ->
    (dot, coff, dop): the statistics in the packed row order [B, Hkv, T, G]
    and dO in the ``pack_heads`` layout, what ``sel_dkdv`` reads."""
    do, o, lse = _contig(do), _contig(o), _contig(lse)
    B, Hq, T, D = o.shape
    rows = B * Hq * T
    G, dop = 1, None
    shape = (B, Hq, T)
    if pack_hkv > 0:
        G = Hq // pack_hkv
        shape = (B, pack_hkv, T, G)
        dop = torch.empty(B, pack_hkv, T, G, D, device=do.device, dtype=do.dtype)
    dot = torch.empty(shape, device=o.device, dtype=torch.float32)
    coff = torch.empty_like(dot)
    _call("nsa_bwd_prep", _lib().nsa_bwd_prep, L.ptr(do), L.ptr(o), None, None, None, None, L.ptr(lse), None, None,
          L.ptr(dot), None, L.ptr(coff), L.ptr(dop), G, T, rows, D, 1, L.dtype_code(do), L.dtype_code(o),
          L.dtype_code(do), _stream(o))
    return (dot, coff) if pack_hkv <= 0 else (dot, coff, dop)


def gate_bwd_prep(do, o_c, o_s, o_w, gate, lse_c, lse_s, lse_w, pack_hkv=0, dgate_f32=False):
    """-> (dot, rowscale, coff [3,B,Hq,T] each, dgate [B,Hq,T,3], dop); branch
    order compression, selection, window; coff = lse * log2(e) -
    log2(rowscale).  With ``pack_hkv`` > 0, dop is dO packed for that many KV
    heads (the ``pack_heads`` layout), else None, and the selection branch's
    dot[1] / rowscale[1] / coff[1] hold their values in the packed row order
    [B, Hkv, T, G] (what ``sel_dkdv`` reads with ``stats_packed``).  The
    branch outputs share one form: dO's dtype, float32 (unrounded) or the
    NSA_F16S form of ``kept_output``.  dgate is in the gate's dtype, or
    float32 (unrounded) with ``dgate_f32``."""
    do, o_c, o_s, o_w, gate = (_contig(t) for t in (do, o_c, o_s, o_w, gate))
    assert o_s.dtype == o_c.dtype and o_w.dtype == o_c.dtype, "branch outputs must share one dtype"
    lse_c, lse_s, lse_w = (_contig(t) for t in (lse_c, lse_s, lse_w))
    B, Hq, T, D = o_c.shape
    rows = B * Hq * T
    dot = torch.empty(3, B, Hq, T, device=o_c.device, dtype=torch.float32)
    rs = torch.empty_like(dot)
    coff = torch.empty_like(dot)
    dgate = torch.empty(gate.shape, device=gate.device, dtype=torch.float32 if dgate_f32 else gate.dtype)
    dop = None
    G = 1
    if pack_hkv > 0:
        G = Hq // pack_hkv
        dop = torch.empty(B, pack_hkv, T, G, D, device=do.device, dtype=do.dtype)
    _call("nsa_bwd_prep", _lib().nsa_bwd_prep, L.ptr(do), L.ptr(o_c), L.ptr(o_s), L.ptr(o_w), L.ptr(gate), L.ptr(dgate),
          L.ptr(lse_c), L.ptr(lse_s), L.ptr(lse_w), L.ptr(dot), L.ptr(rs), L.ptr(coff), L.ptr(dop), G, T, rows, D, 3,
          L.dtype_code(do), L.dtype_code(o_c), L.dtype_code(dgate), _stream(o_c))
    return dot, rs, coff, dgate, dop


def range_dq(mode, q, k, v, kt, do, lse, dot, rowscale, dq, accumulate, window=0, cmp_block=1,
             cmp_stride=1, sel_part=None, sel_idx=None, sel_block=0, out_f32=False):
    """dQ of a range branch into the float32 ``dq`` (added when
    ``accumulate``).  With ``sel_part`` (the selection dQ partials of
    ``sel_dkdv``) and ``sel_idx`` the rows are finished instead: returns
    dq_out in q's dtype = (dq if accumulate) + this branch + the selection
    partials of the valid slots (float32 unrounded with ``out_f32``)."""
    B, Hq, T, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    out = None
    S = 0
    if sel_part is not None:
        S = sel_idx.shape[-1]
        _check_sel_partials(sel_part, q, q.dtype, "sel_part", S=S, block_size=sel_block)
        out = torch.empty(B, Hq, T, D, device=q.device, dtype=torch.float32 if out_f32 else q.dtype)
    _call(_span_name("dq", mode), _lib().nsa_range_dq, mode, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(kt), L.ptr(do),
          L.ptr(lse), L.ptr(dot), L.ptr(rowscale), L.ptr(dq), int(accumulate), B, Hq, Hkv, T, Lk, D,
          int(window), int(cmp_block), int(cmp_stride), L.ptr(sel_part), L.ptr(sel_idx), S, int(sel_block),
          L.ptr(out), L.dtype_code(q), L.dtype_code(out) if out is not None else L.dtype_code(q), _stream(q))
    return out


def range_dq_cw(q, do, kc, vc, ktc, lse_c, dot_c, rs_c, kw, vw, ktw, lse_w, dot_w, rs_w, geom, sel_part, sel_idx,
                out_f32=False):
    """dQ of the compression and window branches in one launch, rows finished
    with the selection dQ partials: returns dq_out in q's dtype (float32
    unrounded with ``out_f32``) = compression + window dQ + the partials of
    the valid slots of ``sel_idx``."""
    B, Hq, T, D = q.shape
    Hkv, Lk = kc.shape[1], kc.shape[2]
    _check_sel_partials(sel_part, q, q.dtype, "sel_part", S=sel_idx.shape[-1], block_size=geom.sel_block)
    out = torch.empty(B, Hq, T, D, device=q.device, dtype=torch.float32 if out_f32 else q.dtype)
    _call("dq[cmp+win]", _lib().nsa_range_dq_cw, L.ptr(q), L.ptr(do), L.ptr(kc), L.ptr(vc), L.ptr(ktc),
          L.ptr(lse_c), L.ptr(dot_c), L.ptr(rs_c), Lk, int(geom.cmp_block), int(geom.cmp_stride), L.ptr(kw),
          L.ptr(vw), L.ptr(ktw), L.ptr(lse_w), L.ptr(dot_w), L.ptr(rs_w), int(geom.window), B, Hq, Hkv, T, D,
          L.ptr(sel_part), L.ptr(sel_idx), sel_idx.shape[-1], int(geom.sel_block), L.ptr(out), L.dtype_code(q),
          L.dtype_code(out), _stream(q))
    return out


# True (default): the chunks of the compression dK/dV and the work items of
# the selection dK/dV write partial rows that a second launch sums in a fixed
# order, so every gradient is bit-identical run to run.  False: they merge
# with float atomics (no partial buffers; the last bits may differ run to run).
DETERMINISTIC_DKDV = True


def range_dkdv(mode, q, k, v, do, coff, dot, window=0, cmp_block=1, cmp_stride=1):
    B, Hq, T, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    dk = torch.empty(B, Hkv, Lk, D, device=q.device, dtype=torch.float32)
    dv = torch.empty_like(dk)
    part, part_bytes = None, 0
    if DETERMINISTIC_DKDV and mode == MODE_COMPRESS:
        part_bytes = int(_lib().nsa_range_dkdv_partial_bytes(mode, B, Hkv, T, Lk, D, int(cmp_block),
                                                             int(cmp_stride), _stream(q)))
        if part_bytes > 0:
            part = torch.empty(part_bytes // 4, device=q.device, dtype=torch.float32)
    _call(_span_name("dkdv", mode), _lib().nsa_range_dkdv, mode, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(do),
          L.ptr(coff), L.ptr(dot), L.ptr(dk), L.ptr(dv), L.ptr(part), part_bytes, B, Hq, Hkv, T, Lk, D,
          int(window), int(cmp_block), int(cmp_stride), L.dtype_code(q), _stream(q))
    return dk, dv


def sel_dq(q, k, v, kt, do, block_idx, block_size, lse, dot, rowscale, dq, accumulate):
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    S = block_idx.shape[-1]
    _call("dq[sel]", _lib().nsa_sel_dq, L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(kt), L.ptr(do), L.ptr(block_idx),
                              L.ptr(lse), L.ptr(dot), L.ptr(rowscale), L.ptr(dq), int(accumulate), B, Hq, Hkv,
                              T, D, S, block_size, L.dtype_code(q), _stream(q))


def csr_device(block_idx, block_size, n_blk=None, pack_slot=False):
    """Block -> query CSR on the GPU without a host sync.

    ``n_blk`` defaults to ``ceil(T / block_size)`` (the trailing partial block
    included, as the selection forward attends to it); the reference grid is
    ``T // block_size`` (nsa_fsa.py:36).  ``pack_slot``: q_of_block holds
    ``(t << ceil(log2 S)) | s`` (query and slot of the pair).  Returns (q_of_block [cap],
    block_offsets [B,Hkv,n_blk+1], pair_bh [cap], pair_count [1]) int32;
    entries past pair_count are unused.
    """
    idx = block_idx.to(torch.int32).contiguous()
    B, Hkv, T, S = idx.shape
    if n_blk is None:
        n_blk = -(-T // block_size)
    cap = B * Hkv * T * S
    dev = idx.device
    q_of_block = torch.empty(max(cap, 1), device=dev, dtype=torch.int32)
    pair_bh = torch.empty(max(cap, 1), device=dev, dtype=torch.int32)
    offsets = torch.empty(B, Hkv, n_blk + 1, device=dev, dtype=torch.int32)
    count = torch.empty(1, device=dev, dtype=torch.int32)
    ws_bytes = int(_lib().nsa_csr_workspace(B, Hkv, T, S, n_blk))
    assert ws_bytes > 0 or cap == 0, "CSR workspace size query failed"
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    _call("nsa_csr_build", _lib().nsa_csr_build, L.ptr(idx), L.ptr(q_of_block), L.ptr(offsets), L.ptr(pair_bh),
          L.ptr(count), L.ptr(ws), ws_bytes, B, Hkv, T, S, block_size, n_blk, int(pack_slot), _stream(idx))
    return q_of_block, offsets, pair_bh, count


def sel_dkdv(q, k, v, do, coff, dot, block_idx, block_size, csr=None, kt=None, want_dq=False, qp=None,
             dop=None, stats_packed=False):
    """dK, dV (float32) of the selection branch over the block -> query CSR;
    with ``want_dq`` also the dQ partials of every (query, slot, pass) for
    ``sel_dq_reduce`` (the CSR must then be built with ``pack_slot``).
    ``qp`` / ``dop``: ``pack_heads`` copies of q / do (made here when not
    given).  ``coff`` / ``dot``: [B, Hq, T], or with ``stats_packed`` already
    in the packed row order [B, Hkv, T, G] (``delta_of(.., pack_hkv)``,
    ``gate_bwd_prep(.., pack_hkv)``), the order the kernel reads."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    if qp is None:
        qp = pack_heads(q, Hkv)
    if dop is None:
        dop = pack_heads(do, Hkv)
    if not stats_packed:
        G = Hq // Hkv
        coff, dot = (t.reshape(B, Hkv, G, T).transpose(2, 3).contiguous() for t in (coff, dot))
    assert coff.numel() == B * Hq * T and dot.numel() == B * Hq * T, "row statistics must cover B*Hq*T rows"
    coff, dot = _contig(coff), _contig(dot)
    idx = block_idx.to(torch.int32).contiguous()
    S = idx.shape[-1]
    if csr is None:
        csr = csr_device(idx, block_size, pack_slot=want_dq)
    q_of_block, offsets, _, count = csr
    dk = torch.empty(B, Hkv, T, D, device=q.device, dtype=torch.float32)
    dv = torch.empty_like(dk)
    dq_part = None
    if want_dq:
        if kt is None:
            kt = transpose_kv(k)
        ns = int(_lib().nsa_sel_partial_slots(S, block_size))
        dq_part = torch.empty(B, Hkv, T, ns, Hq // Hkv, D, device=q.device, dtype=q.dtype)
    ws_bytes = int(_lib().nsa_sel_dkdv_workspace(B, Hkv, T, S, block_size, SEL_DKDV_CHUNK))
    ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
    part, part_bytes = None, 0
    if DETERMINISTIC_DKDV:
        part_bytes = int(_lib().nsa_sel_dkdv_partial_bytes(B, Hkv, T, S, D, block_size, SEL_DKDV_CHUNK))
        part = torch.empty(max(part_bytes // 4, 1), device=q.device, dtype=torch.float32)
    _call("dkdv[sel]", _lib().nsa_sel_dkdv, L.ptr(qp), L.ptr(k), L.ptr(v), L.ptr(kt), L.ptr(dop), L.ptr(coff),
          L.ptr(dot), L.ptr(q_of_block), int(want_dq), L.ptr(offsets),
          L.ptr(count), L.ptr(dk), L.ptr(dv), L.ptr(part), part_bytes, L.ptr(dq_part), L.ptr(ws), ws_bytes, B, Hq,
          Hkv, T, D, S, block_size, SEL_DKDV_CHUNK, L.dtype_code(q), _stream(q))
    return dk, dv, dq_part


def sel_dq_reduce(block_idx, dq_part, dq_acc, block_size, dtype):
    """dQ of the selection branch (+ the float32 ``dq_acc`` of the other
    branches, if given) in ``dtype``.  The kernel reads the partials and
    writes its result in the partials' own dtype (the library cannot see a
    buffer's type: a dtype code that differs from the buffer's would read past
    its end); another ``dtype`` is a conversion of that result."""
    idx = block_idx.to(torch.int32).contiguous()
    B, Hkv, T, S = idx.shape
    G, D = dq_part.shape[-2], dq_part.shape[-1]
    Hq = Hkv * G
    if dq_part.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("selection dQ partials are bfloat16 or float32")
    ns = int(_lib().nsa_sel_partial_slots(S, block_size))
    if not dq_part.is_contiguous() or dq_part.numel() != B * Hkv * T * ns * G * D:
        raise ValueError("dq_part must be the contiguous [B, Hkv, T, slots, G, D] partials of block_idx")
    if dq_acc is not None and (dq_acc.dtype != torch.float32 or dq_acc.numel() != B * Hq * T * D):
        raise TypeError("dq_acc must be a float32 [B, Hq, T, D] accumulator")
    out = torch.empty(B, Hq, T, D, device=dq_part.device, dtype=dq_part.dtype)
    _call("dq[sel]", _lib().nsa_sel_dq_reduce, L.ptr(idx), L.ptr(dq_part), L.ptr(dq_acc), L.ptr(out), B, Hq, Hkv,
          T, D, S, block_size, L.dtype_code(out), _stream(dq_part))
    return out if dtype == out.dtype else out.to(dtype)


def sel_fwd_fsa(q, k, v, block_idx, block_size, csr=None, vt=None, qp=None, o_f32=False):
    """Block-outer selection forward -> (o, lse[f32], csr); ``csr`` is the
    packed block -> query CSR (built here when not given), ``qp`` the
    ``pack_heads`` copy of q (made here when not given).  ``o_f32``: o in
    float32 (unrounded), else in q's dtype."""
    parts, csr = sel_fwd_partials(q, k, v, block_idx, block_size, csr, vt, qp)
    o, lse = sel_merge(block_idx, parts, q.shape, k.shape[1], block_size, o_f32=o_f32)
    return o, lse, csr


def sel_merge(block_idx, parts, q_shape, Hkv, block_size, o_f32=False):
    """The selection output and lse of every row from the partials of
    ``sel_fwd_partials`` (o in the inputs' dtype, or float32 unrounded)."""
    o_part, ml_part = parts
    B, Hq, T, D = q_shape
    idx = block_idx.to(torch.int32).contiguous()
    if o_part.dtype not in (torch.float16, torch.float32) or not o_part.is_contiguous():
        raise TypeError("o_part must be the contiguous fp16 (bf16 inputs) or float32 partials of sel_fwd_partials")
    ns = int(_lib().nsa_sel_partial_slots(idx.shape[-1], block_size))
    if o_part.numel() != B * Hq * T * ns * D or ml_part.numel() != 2 * B * Hq * T * ns \
            or ml_part.dtype != torch.float32 or not ml_part.is_contiguous():
        raise ValueError("o_part / ml_part must hold the [B, Hkv, T, slots, G] partials of block_idx")
    dt = _partial_input_dtype(o_part)
    o = torch.empty(q_shape, device=o_part.device, dtype=torch.float32 if o_f32 else dt)
    lse = torch.empty(B, Hq, T, device=o_part.device, dtype=torch.float32)
    _call("nsa_sel_merge", _lib().nsa_sel_merge, L.ptr(idx), L.ptr(o_part), L.ptr(ml_part), L.ptr(o), L.ptr(lse), B,
          Hq, Hkv, T, D, idx.shape[-1], block_size, L.NSA_BF16 if dt == torch.bfloat16 else L.NSA_F32,
          L.dtype_code(o), _stream(o_part))
    return o, lse


def _partial_dtype(dtype):
    """The selection forward partials' element type for inputs of ``dtype``:
    fp16 for bf16 inputs (11 significant bits; a power-of-two scale per block
    and 64-key pass is folded into each partial's m), the input type
    otherwise."""
    return torch.float16 if dtype == torch.bfloat16 else dtype


def _check_sel_partials(part, q, dtype, what, S=None, block_size=None):
    """A selection partial buffer read by a kernel that takes its element type
    from q: it must be that type, contiguous, and (given S and block_size) of
    the [B, Hkv, T, slots, G, D] size, or the kernel would read another
    buffer's bytes or past its end."""
    if part.dtype != dtype:
        raise TypeError(f"{what} must be {dtype} for {q.dtype} inputs (got {part.dtype})")
    if not part.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if S is not None:
        B, Hq, T, D = q.shape
        ns = int(_lib().nsa_sel_partial_slots(S, block_size))
        if part.numel() != B * Hq * T * ns * D:
            raise ValueError(f"{what} must hold [B, Hkv, T, {ns}, G, D] partials")


def _partial_input_dtype(o_part):
    return torch.bfloat16 if o_part.dtype == torch.float16 else o_part.dtype


def sel_fwd_partials(q, k, v, block_idx, block_size, csr=None, vt=None, qp=None):
    """The block-local selection outputs of every (query, slot, pass):
    -> ((o_part, ml_part), csr), merged by ``sel_fwd_fsa`` or
    ``range_fwd_finish``."""
    check_qkv(q, k, v)
    q, k = _contig(q), _contig(k)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    assert k.shape[2] == T, "selection keys must have the query length"
    assert block_idx.shape[:3] == (B, Hkv, T), "block_idx must be [B, Hkv, T, S]"
    assert block_size >= 16 and block_size % 16 == 0, "block_size must be a multiple of 16"
    idx = block_idx.to(torch.int32).contiguous()
    S = idx.shape[-1]
    if csr is None:
        csr = csr_device(idx, block_size, pack_slot=True)
    if vt is None:
        vt = transpose_kv(v)
    if qp is None:
        qp = pack_heads(q, Hkv)
    q_of_block, offsets, _, _ = csr
    ns = int(_lib().nsa_sel_partial_slots(S, block_size))
    G = Hq // Hkv
    o_part = torch.empty(B, Hkv, T, ns, G, D, device=q.device, dtype=_partial_dtype(q.dtype))
    ml_part = torch.empty(B, Hkv, T, ns, G, 2, device=q.device, dtype=torch.float32)
    ws_bytes = int(_lib().nsa_sel_fwd_bo_workspace(B, Hkv, T, S, block_size, SEL_FWD_CHUNK))
    ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
    _call("fwd[sel]", _lib().nsa_sel_fwd_bo, L.ptr(qp), L.ptr(k), L.ptr(vt), L.ptr(q_of_block), L.ptr(offsets),
          L.ptr(o_part), L.ptr(ml_part), L.ptr(ws), ws_bytes, B, Hq, Hkv, T, D, S, block_size, SEL_FWD_CHUNK,
          L.dtype_code(q), _stream(q))
    return (o_part, ml_part), csr


# ---------------------------------------------------------------------------
# autograd Functions (the reference's boundaries)
# ---------------------------------------------------------------------------

class SelectionAttnHIP(torch.autograd.Function):
    """Selection attention; same boundary as SelectionAttnTriton
    (nsa_selection_backward.py:337-365): saves q, k, v, block_idx, o, lse and
    returns None grads for block_idx / block_size.  Forward and backward run
    block-outer over one packed block -> query CSR built in the forward."""

    @staticmethod
    def forward(ctx, q, k, v, block_idx, block_size):
        q, k, v = _contig(q), _contig(k), _contig(v)
        idx = block_idx.to(torch.int32).contiguous()
        # the backward's row dots dO . o read o unrounded (float32): with the
        # returned bf16 o, a peaked softmax row passes that rounding on to dS
        # and dK (the same choice as the fused layer's branch outputs)
        # the packed Q copy both block-outer kernels read, made once
        qp = pack_heads(q, k.shape[1])
        o32, lse, csr = sel_fwd_fsa(q, k, v, idx, block_size, qp=qp, o_f32=q.dtype != torch.float32)
        o = cast_f32(o32, q.dtype)
        ctx.save_for_backward(q, k, v, idx, o32, lse, qp, *csr)
        ctx.block_size = block_size
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, idx, o, lse, qp, *csr = ctx.saved_tensors
        dq, dk, dv = selection_backward_fsa(q, k, v, idx, ctx.block_size, do, o, lse, csr=tuple(csr), qp=qp)
        return dq, dk, dv, None, None


def selection_backward(q, k, v, block_idx, block_size, do, o, lse=None):
    """dq, dk, dv of the selection branch (input dtypes): dQ query-outer
    (nsa_sel_dq), dK/dV block-outer (the roles of the reference's atomic
    kernel, nsa_selection_backward.py:63-189)."""
    check_qkv(q, k, v)
    q, k, v, do = (_contig(t) for t in (q, k, v, do))
    idx = block_idx.to(torch.int32).contiguous()
    if lse is None:
        _, lse = sel_fwd(q, k, v, idx, block_size)
    dot, coff = delta_of(do, o, lse)
    dq = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    kt = transpose_kv(k)
    sel_dq(q, k, v, kt, do, idx, block_size, lse, dot, None, dq, False)
    dk, dv, _ = sel_dkdv(q, k, v, do, coff, dot, idx, block_size)
    return cast_f32(dq, q.dtype), cast_f32(dk, k.dtype), cast_f32(dv, v.dtype)


def selection_backward_fsa(q, k, v, block_idx, block_size, do, o, lse, csr=None, grads_f32=False, qp=None):
    """dq, dk, dv of the selection branch (input dtypes), all block-outer
    (the roles of selection_backward_fsa, nsa_selection_backward.py:278-334):
    one kernel writes dK/dV and the dQ partials, a reduce sums the partials.
    ``grads_f32``: dk, dv as the float32 sums the kernel forms (not cast).
    ``qp``: the ``pack_heads`` copy of q, if the caller kept it."""
    check_qkv(q, k, v)
    q, k, v, do = (_contig(t) for t in (q, k, v, do))
    idx = block_idx.to(torch.int32).contiguous()
    dot, coff, dop = delta_of(do, o, lse, pack_hkv=k.shape[1])
    dk, dv, dq_part = sel_dkdv(q, k, v, do, coff, dot, idx, block_size, csr=csr, want_dq=True, qp=qp, dop=dop,
                               stats_packed=True)
    dq = sel_dq_reduce(idx, dq_part, None, block_size, q.dtype)
    if grads_f32:
        return dq, dk, dv
    return dq, cast_f32(dk, k.dtype), cast_f32(dv, v.dtype)


class RangeAttnHIP(torch.autograd.Function):
    """Window / compression attention; the boundary of _RangeAttn
    (nsa_fused_kernel.py:521-534).  ``block_size`` is the compression span;
    the optional ``cmp_stride`` (default: block_size) generalises the
    reference's aligned pooling."""

    @staticmethod
    def forward(ctx, q, k, v, mode, window, block_size, cmp_stride=None):
        q, k, v = _contig(q), _contig(k), _contig(v)
        cs = block_size if cmp_stride is None else cmp_stride
        o, lse = range_fwd(mode, q, k, v, window, block_size, cs)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.geo = (mode, window, block_size, cs)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        mode, window, cl, cd = ctx.geo
        dq, dk, dv = range_backward(mode, q, k, v, o, lse, do, window, cl, cd)
        return dq, dk, dv, None, None, None, None


def range_backward(mode, q, k, v, o, lse, do, window=0, cmp_block=1, cmp_stride=1):
    do = _contig(do)
    dot, coff = delta_of(do, o, lse)
    dq = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    kt = transpose_kv(k)
    range_dq(mode, q, k, v, kt, do, lse, dot, None, dq, False, window, cmp_block, cmp_stride)
    dk, dv = range_dkdv(mode, q, k, v, do, coff, dot, window, cmp_block, cmp_stride)
    return cast_f32(dq, q.dtype), cast_f32(dk, k.dtype), cast_f32(dv, v.dtype)


class CompressionWithLse(torch.autograd.Function):
    """Compression attention that also returns its lse (non-differentiable),
    which the importance / top-n kernel consumes."""

    @staticmethod
    def forward(ctx, q, k_cmp, v_cmp, cmp_block, cmp_stride):
        q, k_cmp, v_cmp = _contig(q), _contig(k_cmp), _contig(v_cmp)
        o, lse = range_fwd(MODE_COMPRESS, q, k_cmp, v_cmp, 0, cmp_block, cmp_stride)
        ctx.save_for_backward(q, k_cmp, v_cmp, o, lse)
        ctx.geo = (cmp_block, cmp_stride)
        ctx.mark_non_differentiable(lse)
        return o, lse

    @staticmethod
    def backward(ctx, do, _dlse):
        q, k, v, o, lse = ctx.saved_tensors
        cl, cd = ctx.geo
        dq, dk, dv = range_backward(MODE_COMPRESS, q, k, v, o, lse, do, 0, cl, cd)
        return dq, dk, dv, None, None


def fused_forward(q, kc, vc, ks, vs, kw, vw, gate, block_idx, geom, pooled=False, out_f32=False):
    """The gated three-branch layer's forward (nsa_fused_kernel.py:560-573):
    pool -> compression -> (importance / top-n when block_idx is None) ->
    selection -> window -> gate.  Returns (out, idx, saved): out in q's dtype
    (float32 unrounded with ``out_f32``), the int32 block indices, and the
    tensors ``fused_backward`` needs.  ``pooled``: kc / vc are already the
    pooled compression tokens [B,Hkv,n_cmp,D]."""
    check_qkv(q, kc, vc)
    check_qkv(q, ks, vs)
    check_qkv(q, kw, vw)
    q, kc, vc, ks, vs, kw, vw, gate = (_contig(t) for t in (q, kc, vc, ks, vs, kw, vw, gate))
    T = q.shape[2]
    assert ks.shape[2] == T and kw.shape[2] == T, "selection / window keys must have the query length"
    if pooled:
        assert kc.shape[2] == n_cmp_tokens(T, geom.cmp_block, geom.cmp_stride), \
            "pooled compression keys must have (T - l) // d + 1 tokens"
        k_cmp, v_cmp = kc, vc
    else:
        assert kc.shape[2] == T, "compression keys must have the query length"
        k_cmp = pool_fwd(kc, geom.cmp_block, geom.cmp_stride)
        v_cmp = pool_fwd(vc, geom.cmp_block, geom.cmp_stride)
    S = min(geom.n_sel, T // geom.sel_block) if block_idx is None else block_idx.shape[-1]
    want_sel = S > 0
    qp = (torch.empty(q.shape[0], ks.shape[1], T, q.shape[1] // ks.shape[1], q.shape[3], device=q.device,
                      dtype=q.dtype) if want_sel else torch.empty(0, device=q.device, dtype=q.dtype))
    # the branch outputs stay internal (only their gated sum is returned):
    # they are kept finer than bf16 (fp16 rows with a power-of-two scale per
    # row, or float32 for float32 inputs) so that the backward's row dots
    # dO . o_c see them with 11 significant bits -- with bf16-rounded outputs
    # that dot carries an error that a peaked softmax row passes on to dS, dQ
    # and dK whole
    o_c, lse_c = range_fwd(MODE_COMPRESS, q, k_cmp, v_cmp, 0, geom.cmp_block, geom.cmp_stride,
                           q_packed=qp if want_sel else None, o_kept=want_sel)
    if block_idx is None:
        block_idx = importance_topn(q, k_cmp, lse_c, geom, T)
    idx = block_idx.to(torch.int32).contiguous()
    if idx.shape[-1] > 0:
        # selection partials; the window forward merges them and applies the gate
        parts, csr = sel_fwd_partials(q, ks, vs, idx, geom.sel_block, qp=qp)
        o_w, lse_w, o_s, lse_s, out = range_fwd_finish(q, kw, vw, geom.window, parts, idx, geom.sel_block,
                                                       o_c, gate, out_f32=out_f32)
    else:
        o_s = torch.zeros_like(q)
        lse_s = torch.full(q.shape[:3], -1e9, device=q.device, dtype=torch.float32)
        csr = ()
        o_w, lse_w = range_fwd(MODE_WINDOW, q, kw, vw, geom.window)
        out = gate_fwd(gate, o_c, o_s, o_w)
        if out_f32:
            out = out.float()
    saved = (q, ks, vs, kw, vw, gate, idx, k_cmp, v_cmp, o_c, o_s, o_w, lse_c, lse_s, lse_w, qp, *csr)
    return out, idx, saved


def fused_backward(saved, dout, geom, T, pooled=False, grads_f32=False):
    """The backward of ``fused_forward`` from its ``saved`` tensors ->
    (dq, dkc, dvc, dks, dvs, dkw, dvw, dgate): gate prep, the dQ of the three
    branches, key-side dK/dV per branch, pool backward.  Gradients in the
    input dtype, or float32 (the unrounded values the kernels form) with
    ``grads_f32``."""
    (q, ks, vs, kw, vw, gate, idx, k_cmp, v_cmp, o_c, o_s, o_w,
     lse_c, lse_s, lse_w, qp, *csr) = saved
    dout = _contig(dout)
    dtype = torch.float32 if grads_f32 else q.dtype
    dot, rs, coff, dgate, dop = gate_bwd_prep(dout, o_c, o_s, o_w, gate, lse_c, lse_s, lse_w,
                                              pack_hkv=ks.shape[1] if idx.shape[-1] > 0 else 0,
                                              dgate_f32=grads_f32)
    # one launch walks the compression and window keys of every query and
    # finishes its rows with the selection partials (no float32 dQ buffer)
    fused_dq = FUSE_RANGE_DQ and idx.shape[-1] > 0 and k_cmp.shape[2] > 0
    dq = None if fused_dq else torch.empty(q.shape, device=q.device, dtype=torch.float32)
    # selection dK/dV and dQ partials (block-outer, bound by memory traffic),
    # optionally on a side stream beside the window and compression key-side
    # kernels (bound by MFMA issue) on the current stream
    main = torch.cuda.current_stream(q.device)
    dq_part = None
    side = main
    if idx.shape[-1] > 0:
        side = _side_stream(q.device) if OVERLAP_SEL_BWD else main
        side.wait_stream(main)
        with torch.cuda.stream(side):
            dks, dvs, dq_part = sel_dkdv(q, ks, vs, dout, coff[1], dot[1], idx, geom.sel_block,
                                         csr=tuple(csr), want_dq=True, qp=qp, dop=dop, stats_packed=True)
        # inputs read on the side stream keep their memory until its work is done
        for t in (q, ks, vs, dout, coff, dot, idx, qp, dop, *csr):
            t.record_stream(side)
    else:
        dks = torch.zeros(ks.shape, device=q.device, dtype=torch.float32)
        dvs = torch.zeros_like(dks)
    # window
    kt_w = transpose_kv(kw)
    if not fused_dq:
        range_dq(MODE_WINDOW, q, kw, vw, kt_w, dout, lse_w, dot[2], rs[2], dq, False, geom.window)
    dkw, dvw = range_dkdv(MODE_WINDOW, q, kw, vw, dout, coff[2], dot[2], geom.window)
    # compression dK/dV
    if k_cmp.shape[2] > 0:
        dkp, dvp = range_dkdv(MODE_COMPRESS, q, k_cmp, v_cmp, dout, coff[0], dot[0], 0,
                              geom.cmp_block, geom.cmp_stride)
    else:
        dkp = torch.zeros(k_cmp.shape, device=q.device, dtype=torch.float32)
        dvp = torch.zeros_like(dkp)
    if dq_part is not None and side is not main:
        main.wait_stream(side)
        for t in (dks, dvs, dq_part):
            t.record_stream(main)
    # compression dQ; it finishes the rows: window dQ + its own + the
    # selection partials, written in the output dtype
    if k_cmp.shape[2] > 0:
        kt_c = transpose_kv(k_cmp)
        if fused_dq:
            dq_out = range_dq_cw(q, dout, k_cmp, v_cmp, kt_c, lse_c, dot[0], rs[0], kw, vw, kt_w, lse_w, dot[2],
                                 rs[2], geom, dq_part, idx, out_f32=grads_f32)
        elif dq_part is not None and SEPARATE_SEL_DQ:
            range_dq(MODE_COMPRESS, q, k_cmp, v_cmp, kt_c, dout, lse_c, dot[0], rs[0], dq, True, 0,
                     geom.cmp_block, geom.cmp_stride)
            dq_out = sel_dq_reduce(idx, dq_part, dq, geom.sel_block, q.dtype).to(dtype)
        elif dq_part is not None:
            dq_out = range_dq(MODE_COMPRESS, q, k_cmp, v_cmp, kt_c, dout, lse_c, dot[0], rs[0], dq, True, 0,
                              geom.cmp_block, geom.cmp_stride, sel_part=dq_part, sel_idx=idx,
                              sel_block=geom.sel_block, out_f32=grads_f32)
        else:
            range_dq(MODE_COMPRESS, q, k_cmp, v_cmp, kt_c, dout, lse_c, dot[0], rs[0], dq, True, 0,
                     geom.cmp_block, geom.cmp_stride)
            dq_out = cast_f32(dq, dtype)
    else:
        # (the reduce writes the partials' dtype)
        dq_out = (sel_dq_reduce(idx, dq_part, dq, geom.sel_block, q.dtype).to(dtype) if dq_part is not None
                  else cast_f32(dq, dtype))
    if pooled:
        dkc, dvc = cast_f32(dkp, dtype), cast_f32(dvp, dtype)
    else:
        dkc = pool_bwd(dkp, T, geom.cmp_block, geom.cmp_stride, dtype)
        dvc = pool_bwd(dvp, T, geom.cmp_block, geom.cmp_stride, dtype)
    return (dq_out, dkc, dvc, cast_f32(dks, dtype), cast_f32(dvs, dtype),
            cast_f32(dkw, dtype), cast_f32(dvw, dtype), dgate)


def fused_capi(q, kc, vc, ks, vs, kw, vw, gate, geom, dout, block_idx=None, pooled=False):
    """The layer through the two C entry points a C caller runs,
    ``nsa_fused_fwd`` and ``nsa_fused_bwd`` (one call each, caller-owned ctx
    and scratch buffers) -> (out, block_idx, (dq, dkc, dvc, dks, dvs, dkw,
    dvw, dgate))."""
    q, kc, vc, ks, vs, kw, vw, gate, dout = (_contig(t) for t in (q, kc, vc, ks, vs, kw, vw, gate, dout))
    B, Hq, T, D = q.shape
    Hkv = ks.shape[1]
    dt = L.dtype_code(q)
    dims = (B, Hq, Hkv, T, D, geom.cmp_block, geom.cmp_stride, geom.sel_block, geom.n_sel, geom.window)
    ctx_bytes = int(_lib().nsa_fused_ctx_bytes(*dims, int(pooled), dt))
    scr_bytes = int(_lib().nsa_fused_scratch_bytes(*dims, int(pooled), dt, _stream(q)))
    assert ctx_bytes > 0 and scr_bytes > 0, "nsa_fused: unsupported shape (T must reach cmp_block and sel_block)"
    ctx = torch.empty(ctx_bytes, device=q.device, dtype=torch.uint8)
    scratch = torch.empty(scr_bytes, device=q.device, dtype=torch.uint8)
    S = min(geom.n_sel, T // geom.sel_block)
    given = block_idx is not None
    idx = (block_idx.to(torch.int32).contiguous() if given
           else torch.empty(B, Hkv, T, S, device=q.device, dtype=torch.int32))
    out = torch.empty_like(q)
    _call("nsa_fused_fwd", _lib().nsa_fused_fwd, *map(L.ptr, (q, kc, vc, ks, vs, kw, vw, gate)), L.ptr(idx),
          int(given), L.ptr(out), L.ptr(ctx), ctx_bytes, L.ptr(scratch), scr_bytes, *dims, int(geom.force_init),
          int(geom.n_local), int(pooled), dt, _stream(q))
    grads = [torch.empty_like(t) for t in (q, kc, vc, ks, vs, kw, vw, gate)]
    _call("nsa_fused_bwd", _lib().nsa_fused_bwd, *map(L.ptr, (dout, q, kc, vc, ks, vs, kw, vw, gate)), L.ptr(idx),
          L.ptr(ctx), ctx_bytes, L.ptr(scratch), scr_bytes, *map(L.ptr, grads), *dims, int(pooled), dt, _stream(q))
    return out, idx, tuple(grads)


class NSAFusedHIP(torch.autograd.Function):
    """All three gated branches in one boundary (nsa_fused_kernel.py:560-573):
    ``fused_forward`` and ``fused_backward``.  Same outputs and gradients as
    composing the per-branch Functions.

    With ``pooled=True`` the compression inputs ``kc``/``vc`` are already the
    pooled tokens ``[B,Hkv,n_cmp,D]`` (the learned BlockCompressor of the
    model path, nsa_model.py:334-337) and receive their gradients directly.
    """

    @staticmethod
    def forward(ctx, q, kc, vc, ks, vs, kw, vw, gate, block_idx, geom, pooled=False):
        out, idx, saved = fused_forward(q, kc, vc, ks, vs, kw, vw, gate, block_idx, geom, pooled)
        ctx.save_for_backward(*saved)
        ctx.geom = geom
        ctx.T = q.shape[2]
        ctx.pooled = pooled
        ctx.mark_non_differentiable(idx)
        return out, idx

    @staticmethod
    def backward(ctx, dout, _didx):
        grads = fused_backward(ctx.saved_tensors, dout, ctx.geom, ctx.T, ctx.pooled)
        return (*grads, None, None, None)


class NSAFusedCAPI(torch.autograd.Function):
    """``NSAFusedHIP``'s layer through the two C entry points a C caller runs
    (``nsa_fused_fwd`` / ``nsa_fused_bwd``): the same kernels with the same
    arguments (bit-identical outputs and gradients), issued from C++ in one
    library call per direction instead of the Python sequence of about a dozen
    calls and their allocations.  Caller-owned buffers: the saved context
    (branch outputs, lse, packed Q, CSR) lives from the forward to the
    backward; each call takes its own scratch."""

    @staticmethod
    def forward(ctx, q, kc, vc, ks, vs, kw, vw, gate, block_idx, geom, pooled=False):
        check_qkv(q, ks, vs)
        check_qkv(q, kw, vw)
        ins = tuple(_contig(t) for t in (q, kc, vc, ks, vs, kw, vw, gate))
        q = ins[0]
        B, Hq, T, D = q.shape
        Hkv = ins[3].shape[1]
        dt = L.dtype_code(q)
        dims = (B, Hq, Hkv, T, D, geom.cmp_block, geom.cmp_stride, geom.sel_block, geom.n_sel, geom.window)
        ctx_bytes = int(_lib().nsa_fused_ctx_bytes(*dims, int(pooled), dt))
        scr_bytes = int(_lib().nsa_fused_scratch_bytes(*dims, int(pooled), dt, _stream(q)))
        assert ctx_bytes > 0 and scr_bytes > 0, "nsa_fused: unsupported shape (T must reach cmp_block and sel_block)"
        saved = torch.empty(ctx_bytes, device=q.device, dtype=torch.uint8)
        scratch = torch.empty(scr_bytes, device=q.device, dtype=torch.uint8)
        S = min(geom.n_sel, T // geom.sel_block)
        given = block_idx is not None
        idx = (block_idx.to(torch.int32).contiguous() if given
               else torch.empty(B, Hkv, T, S, device=q.device, dtype=torch.int32))
        out = torch.empty_like(q)
        _call("nsa_fused_fwd", _lib().nsa_fused_fwd, *map(L.ptr, ins), L.ptr(idx), int(given), L.ptr(out),
              L.ptr(saved), ctx_bytes, L.ptr(scratch), scr_bytes, *dims, int(geom.force_init), int(geom.n_local),
              int(pooled), dt, _stream(q))
        ctx.save_for_backward(*ins, idx, saved)
        ctx.meta = (dims, scr_bytes, int(pooled), dt)
        ctx.mark_non_differentiable(idx)
        return out, idx

    @staticmethod
    def backward(ctx, dout, _didx):
        *ins, idx, saved = ctx.saved_tensors
        dims, scr_bytes, pooled, dt = ctx.meta
        dout = _contig(dout.to(ins[0].dtype))
        scratch = torch.empty(scr_bytes, device=dout.device, dtype=torch.uint8)
        grads = [torch.empty_like(t) for t in ins]
        _call("nsa_fused_bwd", _lib().nsa_fused_bwd, L.ptr(dout), *map(L.ptr, ins), L.ptr(idx), L.ptr(saved),
              saved.numel(), L.ptr(scratch), scr_bytes, *map(L.ptr, grads), *dims, pooled, dt, _stream(dout))
        return (*grads, None, None, None)


# True: a model layer (nsa_attention_layer) runs through the C entry points
LAYER_CAPI = True


def nsa_attention_layer(q, kc, vc, ks, vs, kw, vw, gate_logits, geom: NSAGeometry, block_idx=None, pooled=False):
    """``nsa_attention`` for a model layer: through the C entry points
    (``NSAFusedCAPI``) where they take the shape, one launch sequence per
    direction issued from C++; else (``T`` shorter than a compression or
    selection block, per-call timing wanted, or ``LAYER_CAPI`` off) through
    ``NSAFusedHIP``."""
    T = q.shape[2]
    if LAYER_CAPI and _TIMER is None and T >= geom.cmp_block and T >= geom.sel_block:
        return NSAFusedCAPI.apply(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, geom, pooled)
    return NSAFusedHIP.apply(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, geom, pooled)


def nsa_attention(q, kc, vc, ks, vs, kw, vw, gate_logits, geom: NSAGeometry, block_idx=None, pooled=False):
    """Full NSA attention (pre out-projection) on the HIP path.

    With ``block_idx=None`` the block choice comes from the compression
    importance and top-n (nsa_model.py:343-355) computed on the GPU.
    ``pooled=True``: ``kc``/``vc`` are pooled compression tokens.
    Returns ``(out, block_idx)``.
    """
    return NSAFusedHIP.apply(q, kc, vc, ks, vs, kw, vw, gate_logits, block_idx, geom, pooled)


# ---------------------------------------------------------------------------
# compression phi (NSA paper eq. 7): an MLP over each span of l tokens
# ---------------------------------------------------------------------------

class PhiCompressHIP(torch.autograd.Function):
    """``out[b,h,i] = W2 silu(W1 vec(x[b,h,i d : i d + l] + P) + b1) + b2``
    for ``x [B,H,T,D]``: the forward, the hidden-layer backward and the
    parameter gradients (float32 sums in a fixed order) on HIP kernels that
    read the overlapping spans in place.  Parameters may be float32
    (autocast): the kernels take W1 / W2 in x's dtype, biases in float32."""

    @staticmethod
    def forward(ctx, x, pos, w1, b1, w2, b2, l, d):
        x = _contig(x)
        B, Hh, T, D = x.shape
        Hd = w1.shape[0]
        assert w1.shape == (Hd, l * D) and w2.shape == (D, Hd) and pos.shape == (l, D), "phi: parameter shapes"
        assert b1.shape == (Hd,) and b2.shape == (D,)
        n = n_cmp_tokens(T, l, d)
        dt = x.dtype
        with torch.autocast("cuda", enabled=False):
            c1 = (b1.float() + w1.float() @ pos.float().reshape(-1)).contiguous()
        w1c, w2c = _contig(w1.to(dt)), _contig(w2.to(dt))
        out = torch.empty(B, Hh, n, D, device=x.device, dtype=dt)
        pre = torch.empty(B * Hh * n, Hd, device=x.device, dtype=torch.float32)
        if n > 0:
            _call("nsa_phi_fwd", _lib().nsa_phi_fwd, L.ptr(x), L.ptr(w1c), L.ptr(c1), L.ptr(w2c),
                  L.ptr(b2.float().contiguous()), L.ptr(out), L.ptr(pre), B * Hh, T, D, Hd, l, d, L.dtype_code(x),
                  _stream(x))
        ctx.save_for_backward(x, pos, w1, b1, w2, b2, pre)
        ctx.geom = (l, d)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, pos, w1, b1, w2, b2, pre = ctx.saved_tensors
        l, d = ctx.geom
        B, Hh, T, D = x.shape
        Hd = w1.shape[0]
        n = n_cmp_tokens(T, l, d)
        BH, M = B * Hh, B * Hh * n
        dx = torch.zeros_like(x)
        if n == 0:
            return (dx, torch.zeros_like(pos), torch.zeros_like(w1), torch.zeros_like(b1), torch.zeros_like(w2),
                    torch.zeros_like(b2), None, None)
        dout = _contig(dout.to(x.dtype))
        w2t = _contig(w2.to(x.dtype).t())
        dpre = torch.empty(M, Hd, device=x.device, dtype=torch.float32)
        _call("nsa_phi_dpre", _lib().nsa_phi_dpre, L.ptr(dout), L.ptr(w2t), L.ptr(pre), L.ptr(dpre), BH, n, D, Hd,
              L.dtype_code(x), _stream(x))
        # parameter gradients summed in float32 (a bf16 result would round
        # each entry of a sum over every span), in a fixed order; the span
        # gradient, which the fold adds at most ceil(l / d) at a time in
        # float, runs in x's dtype
        f32 = dict(device=x.device, dtype=torch.float32)
        dw1, db1 = torch.empty(Hd, l * D, **f32), torch.empty(Hd, **f32)
        dw2, db2, dpos = torch.empty(D, Hd, **f32), torch.empty(D, **f32), torch.empty(l, D, **f32)
        ws_bytes = int(_lib().nsa_phi_wgrad_workspace(BH, n, D, Hd, l))
        assert ws_bytes > 0, "phi: unsupported shape for the weight gradients"
        ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
        pos32, w132 = _contig(pos.float()), _contig(w1.float())
        _call("nsa_phi_wgrad", _lib().nsa_phi_wgrad, L.ptr(x), L.ptr(dout), L.ptr(dpre), L.ptr(pre), L.ptr(pos32),
              L.ptr(w132), L.ptr(dw1), L.ptr(db1), L.ptr(dw2), L.ptr(db2), L.ptr(dpos), L.ptr(ws), ws_bytes, BH, T,
              D, Hd, l, d, L.dtype_code(x), _stream(x))
        with torch.autocast("cuda", enabled=False):
            dspan = dpre.to(x.dtype) @ w1.to(x.dtype)
        _call("nsa_phi_fold", _lib().nsa_phi_fold, L.ptr(dspan), L.dtype_code(dspan), L.ptr(dx), BH, T, D, l, d,
              L.dtype_code(x), _stream(x))
        return (dx, dpos.to(pos.dtype), dw1.to(w1.dtype), db1.to(b1.dtype), dw2.to(w2.dtype), db2.to(b2.dtype),
                None, None)


def phi_compress(x, pos, w1, b1, w2, b2, l, d):
    """Pooled tokens ``[B,H,n,D]`` of ``x [B,H,T,D]`` through phi (span l, stride d)."""
    return PhiCompressHIP.apply(x, pos, w1, b1, w2, b2, l, d)


# ---------------------------------------------------------------------------
# decode: one new query per sequence against its KV caches (no reference
# counterpart; row t = lens[b] - 1 of NSAAttention.forward, nsa_model.py:196-304)
# ---------------------------------------------------------------------------

def decode_workspace_bytes(B, Hq, Hkv, D, Tcap, Ncap, geom: NSAGeometry):
    n = int(_lib().nsa_decode_workspace(B, Hq, Hkv, D, Tcap, Ncap, geom.cmp_block, geom.cmp_stride,
                                        geom.sel_block, geom.n_sel, geom.window))
    assert n > 0, "decode: unsupported shape (head dim, capacities or candidate blocks)"
    return n


def decode_fwd(q, k_cmp, v_cmp, ks, vs, kw, vw, gate, lens, geom: NSAGeometry, return_scores=False,
               return_branches=False, workspace=None):
    """One decode step for every sequence: ``q [B,Hq,D]`` and ``gate
    [B,Hq,3]`` are the new tokens' query and gate logits, ``lens`` (int32
    [B], on the device) the cache lengths including the new token.  Caches:
    ``k_cmp/v_cmp [B,Hkv,Ncap,D]`` pooled, ``ks..vw [B,Hkv,Tcap,D]``.

    Returns ``(out [B,Hq,D], block_idx [B,Hkv,n_sel])`` (-1 past the
    sequence's S), plus a dict with ``scores`` (raw importance of candidate
    blocks, float32 ``[B,Hkv,(Tcap-1)//sel_block+1]``, NaN past the
    candidates) and/or ``o_branch`` ``[3,B,Hq,D]`` / ``lse_branch`` ``[3,B,Hq]``
    (compression, selection, window) when asked.
    """
    assert q.dim() == 3 and q.is_cuda, "decode: q must be [B, Hq, D] on the GPU"
    B, Hq, D = q.shape
    caches = [_contig(x) for x in (ks, vs, kw, vw)]
    assert ks.dim() == 4 and ks.shape[0] == B and ks.shape[3] == D, "decode: caches must be [B, Hkv, Tcap, D]"
    Hkv, Tcap = ks.shape[1], ks.shape[2]
    assert Hq % Hkv == 0, "GQA needs n_q_heads divisible by n_kv_heads"
    for x in caches:
        assert x.shape == ks.shape and x.dtype == q.dtype, "decode: branch caches differ in shape or dtype"
    k_cmp, v_cmp = _contig(k_cmp), _contig(v_cmp)
    Ncap = k_cmp.shape[2]
    assert k_cmp.shape == (B, Hkv, Ncap, D) and v_cmp.shape == k_cmp.shape, "decode: pooled caches [B, Hkv, Ncap, D]"
    assert k_cmp.dtype == q.dtype and v_cmp.dtype == q.dtype
    assert gate.shape == (B, Hq, 3) and gate.dtype == q.dtype, "decode: gate logits [B, Hq, 3] in q's dtype"
    assert lens.dtype == torch.int32 and lens.shape == (B,) and lens.is_cuda, "decode: lens int32 [B] on the GPU"
    q, gate, lens = _contig(q), _contig(gate), _contig(lens)
    nbytes = decode_workspace_bytes(B, Hq, Hkv, D, Tcap, Ncap, geom)
    if workspace is None:
        workspace = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    assert workspace.numel() * workspace.element_size() >= nbytes and workspace.data_ptr() % 256 == 0, \
        "decode: workspace too small or not 256-byte aligned"
    out = torch.empty_like(q)
    idx = torch.empty(B, Hkv, geom.n_sel, device=q.device, dtype=torch.int32)
    ncand_cap = (Tcap - 1) // geom.sel_block + 1
    scores = (torch.full((B, Hkv, ncand_cap), float("nan"), device=q.device, dtype=torch.float32)
              if return_scores else None)
    o_br = torch.empty(3, B, Hq, D, device=q.device, dtype=torch.float32) if return_branches else None
    lse_br = torch.empty(3, B, Hq, device=q.device, dtype=torch.float32) if return_branches else None
    _call("nsa_decode_fwd", _lib().nsa_decode_fwd, L.ptr(q), L.ptr(k_cmp), L.ptr(v_cmp), *map(L.ptr, caches),
          L.ptr(gate), L.ptr(lens), L.ptr(out), L.ptr(idx), L.ptr(scores), L.ptr(o_br), L.ptr(lse_br),
          L.ptr(workspace), workspace.numel() * workspace.element_size(), B, Hq, Hkv, D, Tcap, Ncap,
          geom.cmp_block, geom.cmp_stride, geom.sel_block, geom.n_sel, geom.window, int(geom.force_init),
          geom.n_local, L.dtype_code(q), _stream(q))
    if not (return_scores or return_branches):
        return out, idx
    extras = {}
    if return_scores:
        extras["scores"] = scores
    if return_branches:
        extras["o_branch"], extras["lse_branch"] = o_br, lse_br
    return out, idx, extras


def decode_append(kc, vc, ks, vs, kw, vw, k_cmp, v_cmp, new_rows, lens, geom: NSAGeometry):
    """Write one token per sequence into the caches (in place): ``new_rows``
    are the six ``[B,Hkv,D]`` rows (kc vc ks vs kw vw) for position
    ``lens[b]``; a pooled token is added when the new length completes a
    span.  Returns the new lengths (a new int32 tensor; full caches keep
    theirs)."""
    caches = (kc, vc, ks, vs, kw, vw)
    B, Hkv, Tcap, D = kc.shape
    for x in caches + (k_cmp, v_cmp):
        assert x.is_contiguous() and x.dtype == kc.dtype, "decode_append: caches must be contiguous, one dtype"
    for x in caches:
        assert x.shape == kc.shape
    assert k_cmp.shape[:2] == (B, Hkv) and k_cmp.shape[3] == D and v_cmp.shape == k_cmp.shape
    rows = [_contig(r) for r in new_rows]
    assert len(rows) == 6 and all(r.shape == (B, Hkv, D) and r.dtype == kc.dtype for r in rows)
    assert lens.dtype == torch.int32 and lens.shape == (B,) and lens.is_contiguous()
    lens_out = torch.empty_like(lens)
    _call("nsa_decode_append", _lib().nsa_decode_append, *map(L.ptr, caches), L.ptr(k_cmp), L.ptr(v_cmp),
          *map(L.ptr, rows), L.ptr(lens), L.ptr(lens_out), B, Hkv, D, Tcap, k_cmp.shape[2], geom.cmp_block,
          geom.cmp_stride, L.dtype_code(kc), _stream(kc))
    return lens_out
