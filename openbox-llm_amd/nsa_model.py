"""NSA attention, its dense control arm and a small decoder around them, with
the reference's ``attn_impl`` switch (drop-in for the reference module
nsa_model.py).

* ``NSAAttention(attn_impl='ref')``: the dense torch definition of the layer
  (nsa_model.py:196-304): three masked ``[B,Hq,T,T]`` attentions over the same
  projections.  It runs on any device and is the definition the fused path is
  checked against.
* ``NSAAttention(attn_impl='fused')``: the same layer with the attention on
  the MI355X HIP kernels: compression attention over the learned pooled
  tokens, block importance + top-n, selection, sliding window and the gate
  blend in one autograd boundary (``nsa_hip_ops.NSAFusedHIP``).  The library
  is loaded on first use and its absence raises; nothing falls back to the
  'ref' path.
* ``FullAttention``, ``make_attention``, ``Block``, ``NSATransformer``,
  ``branch_of``, ``param_groups``, ``REQUIRED_BRANCHES``: the model the
  reference's training scripts build (nsa_model.py:377-549), so that
  ``from nsa_model import NSATransformer`` keeps working with this directory
  first on ``sys.path``.

Parameters, their names and their initialisation follow the reference
(nsa_model.py:147-195, :435-476), so a reference ``state_dict`` loads
unchanged.  With its defaults the block grid is the reference's aligned one:
compression and selection share ``block_size`` and pooled token j summarises
block j.  Block choice in both paths ranks blocks by descending importance
and, among equal scores, by ascending block index.  The reference's
``torch.topk`` leaves that order open; it only matters on rows with fewer
complete blocks than ``n_selected_blocks``, where the masked fillers tie.
``forward(x, block_idx=...)`` takes an explicit block choice ``[B,Hkv,T,S]``
(-1 = empty slot) instead, e.g. one recorded from the reference.

Keyword-only extensions, off by default (none is in the reference):

* NSA geometry of the BASELINE configurations: ``cmp_stride`` (compression
  span ``block_size`` slid by ``cmp_stride``: overlapping pooled tokens),
  ``sel_block`` (selection block size; block importance collects the pooled
  tokens by span overlap, the NSA paper's eq. 9), ``force_init`` /
  ``n_local`` (block 0 and the ``n_local`` most recent blocks always chosen).
* ``compressor='mlp'``: the NSA paper's compression phi (``MLPCompressor``,
  a learnable MLP over each span with an intra-block position encoding) in
  place of the reference's weighted mean + linear; the fused path runs it on
  the HIP kernels.
* model variants for a Llama-style decoder: ``norm='rms'`` (RMSNorm),
  ``ffn='swiglu'`` with ``ffn_hidden``, ``pos='rope'`` (rotary position on
  queries and keys of every branch, keys rotated before pooling),
  ``tie_embeddings``, ``dense_impl='sdpa'`` (the dense arm through
  ``torch.nn.functional.scaled_dot_product_attention``).
"""


import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint

__all__ = ["masked_softmax", "expand_kv", "BlockCompressor", "MLPCompressor", "NSAAttention", "FullAttention", "make_attention",
           "Block", "NSATransformer", "branch_of", "param_groups", "REQUIRED_BRANCHES", "Rotary", "SwiGLU"]


def masked_softmax(scores, keep_mask):
    """Softmax over the last dim restricted to ``keep_mask``; rows with no kept
    position come out as zeros (nsa_model.py:70-82)."""
    filled = scores.masked_fill(~keep_mask, torch.finfo(scores.dtype).min)
    return torch.softmax(filled, dim=-1) * keep_mask.any(dim=-1, keepdim=True)


def expand_kv(x, group_size):
    """``[B,Hkv,S,D] -> [B,Hkv*G,S,D]``; query head h reads KV head h // G
    (nsa_model.py:85-93)."""
    return x.repeat_interleave(group_size, dim=1)


def _scores(q, k, scale):
    """``q @ k^T * scale`` with the transposed operand made contiguous (batched
    bf16 products with a transposed right operand are avoided on this GPU)."""
    return torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale


_SPLITK_PARTS = 16
_SPLITK_PART_BYTES = 80 << 20    # float32 partials of one split-K product: fewer parts past this
_SPLITK_MAX_BYTES = 256 << 20    # ... and no split past this


def _weight_grad(g2, x2):
    """``g2^T x2`` for the rows of a linear layer ([M, out], [M, in]).  On the
    GPU in 16 bits, with M in the tens of thousands, one GEMM of a small
    [out, in] result over M runs on a few dozen workgroups; the rows are taken
    instead as 16 batched products with float32 outputs (bmm's out_dtype),
    summed in float32: 2.5-3x faster at the c4 shapes.  Large outputs take 8
    parts, as the extra partials' sum costs more than the parallelism gains
    there ([2048, 768]: 118 us at 8 parts, 145 at 16, 229 as one GEMM).  Either
    way the weight gradient comes out in float32, with no bf16 rounding."""
    M, P = g2.shape[0], _SPLITK_PARTS
    if not (g2.is_cuda and g2.dtype in (torch.bfloat16, torch.float16)):
        return g2.t() @ x2
    while P > 8 and P * g2.shape[1] * x2.shape[1] * 4 > _SPLITK_PART_BYTES:
        P //= 2
    if M % P == 0 and M >= P * 64 and P * g2.shape[1] * x2.shape[1] * 4 <= _SPLITK_MAX_BYTES:
        return torch.bmm(g2.view(P, M // P, -1).transpose(1, 2), x2.view(P, M // P, -1),
                         out_dtype=torch.float32).sum(0)
    return torch.mm(g2.t(), x2, out_dtype=torch.float32)


class _SplitKLinear(torch.autograd.Function):
    """``F.linear`` in the compute dtype ``cdt`` (inputs cast as autocast
    would), with the weight gradient through ``_weight_grad``.  Saves the cast
    input and weight, as autocast's linear does."""

    @staticmethod
    def forward(ctx, x, w, b, cdt):
        xc, wc = x.to(cdt), w.to(cdt)
        ctx.save_for_backward(xc, wc)
        ctx.meta = (x.dtype, w.dtype, None if b is None else b.dtype)
        with torch.autocast("cuda", enabled=False):
            return F.linear(xc, wc, None if b is None else b.to(cdt))

    @staticmethod
    def backward(ctx, g):
        xc, wc = ctx.saved_tensors
        x_dt, w_dt, b_dt = ctx.meta
        g2 = g.reshape(-1, g.shape[-1]).to(wc.dtype)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = (g2 @ wc).view(*xc.shape[:-1], wc.shape[1]).to(x_dt)
        if ctx.needs_input_grad[1]:
            dw = _weight_grad(g2, xc.reshape(-1, xc.shape[-1])).to(w_dt)
        if b_dt is not None and ctx.needs_input_grad[2]:
            db = g2.float().sum(0).to(b_dt)
        return dx, dw, db, None


def _linear(x, w, b=None):
    """``F.linear(x, w, b)``; on the GPU with a 16-bit compute dtype (autocast,
    or 16-bit x and w) through ``_SplitKLinear``."""
    if x.is_cuda:
        if torch.is_autocast_enabled("cuda"):
            cdt = torch.get_autocast_dtype("cuda")
            if cdt in (torch.bfloat16, torch.float16):
                return _SplitKLinear.apply(x, w, b, cdt)
        elif x.dtype in (torch.bfloat16, torch.float16) and w.dtype == x.dtype:
            return _SplitKLinear.apply(x, w, b, x.dtype)
    return F.linear(x, w, b)


class Linear(nn.Linear):
    """``nn.Linear`` (same parameters and state_dict names) computed by
    ``_linear``."""

    def forward(self, x):
        return _linear(x, self.weight, self.bias)


class BlockCompressor(nn.Module):
    """Learned pooling of one span of ``block_size`` tokens into one token:
    ``proj(sum_p softmax(pool_logits)_p * (x_p + intra_pos_p))``
    (nsa_model.py:100-123).  ``pool_logits`` start at zero, i.e. a plain mean."""

    def __init__(self, block_size, d_head):
        super().__init__()
        self.block_size = block_size
        self.intra_pos = nn.Parameter(torch.zeros(block_size, d_head))
        self.pool_logits = nn.Parameter(torch.zeros(block_size))
        self.proj = Linear(d_head, d_head, bias=False)

    def forward(self, x_blocks):
        """``x_blocks [B,Hkv,n_blk,block_size,D] -> [B,Hkv,n_blk,D]``."""
        w = torch.softmax(self.pool_logits, dim=0)
        pooled = ((x_blocks + self.intra_pos) * w[:, None]).sum(dim=-2)
        return self.proj(pooled)

    def pool_sequence(self, x, stride):
        """The same pooled tokens straight from ``x [B,Hkv,T,D]`` (spans
        ``[i stride, i stride + block_size)``) on the HIP kernels, which read
        the overlapping spans in place; the weighted sum in float32, as the
        unfolded form computes it, the projection under the caller's
        autocast (its weight gradient split over the pooled tokens)."""
        import nsa_hip_ops as ops
        w = torch.softmax(self.pool_logits, dim=0)
        return _linear(ops.weighted_pool(x, w, self.intra_pos, self.block_size, stride), self.proj.weight)


class MLPCompressor(nn.Module):
    """The NSA paper's compression phi (arXiv:2502.11089, eq. 7): a learnable
    MLP with an intra-block position encoding maps a span of ``block_size``
    tokens to one token, ``fc2(silu(fc1(vec(x_span + intra_pos))))``.  It is
    the paper-faithful alternative to ``BlockCompressor`` (the reference's
    weighted mean + linear, nsa_model.py:100-123); ``hidden`` defaults to the
    head dim.  ``pool_sequence`` computes the same pooled tokens on the MI355X
    kernels straight from ``[B,Hkv,T,D]`` (the overlapping spans are read in
    place)."""

    def __init__(self, block_size, d_head, hidden=None):
        super().__init__()
        self.block_size = block_size
        self.hidden = d_head if hidden is None else hidden
        self.intra_pos = nn.Parameter(torch.zeros(block_size, d_head))
        self.fc1 = Linear(block_size * d_head, self.hidden)
        self.fc2 = Linear(self.hidden, d_head)

    def forward(self, x_blocks):
        """``x_blocks [B,Hkv,n_blk,block_size,D] -> [B,Hkv,n_blk,D]``."""
        z = (x_blocks + self.intra_pos).flatten(-2)
        return self.fc2(F.silu(self.fc1(z)))

    def pool_sequence(self, x, stride):
        """``x [B,Hkv,T,D] -> [B,Hkv,n,D]``, spans ``[i stride, i stride +
        block_size)``, on the HIP kernels."""
        import nsa_hip_ops as ops
        return ops.phi_compress(x, self.intra_pos, self.fc1.weight, self.fc1.bias, self.fc2.weight, self.fc2.bias,
                                self.block_size, stride)


class Rotary(nn.Module):
    """Rotary position embedding (RoFormer, arXiv:2104.09864) in the half-split
    layout: the first and second halves of the head dim form the rotated
    pairs, with frequencies ``base ** (-2i / dim)``."""

    def __init__(self, dim, base=10000.0):
        super().__init__()
        assert dim % 2 == 0, "rotary needs an even head dim"
        inv = base ** (-torch.arange(0, dim, 2, dtype=torch.float64) / dim)
        self.register_buffer("inv_freq", inv.float(), persistent=False)
        self._tables = {}

    def tables(self, T, device, dtype):
        """The factors ``forward`` multiplies by, ``cos, sin [T, dim/2]`` with
        the values of ``dtype``, held as float32 (the fused head split's
        tables); cached per length, device, dtype and frequency buffer."""
        inv = self.inv_freq
        key = (T, str(device), dtype, inv.dtype, inv.data_ptr(), inv._version)
        hit = self._tables.get(key)
        if hit is None:
            with torch.no_grad(), torch.autocast(device_type=torch.device(device).type, enabled=False):
                ang = torch.arange(T, device=device, dtype=torch.float32)[:, None] * inv.to(device)[None, :]
                hit = (ang.cos().to(dtype).float().contiguous(), ang.sin().to(dtype).float().contiguous())
            if len(self._tables) > 8:
                self._tables.clear()
            self._tables[key] = hit
        return hit

    def forward(self, x):
        """``x [B,H,T,D]`` rotated by position ``t``."""
        T = x.shape[2]
        ang = torch.arange(T, device=x.device, dtype=torch.float32)[:, None] * self.inv_freq[None, :]
        cos, sin = ang.cos().to(x.dtype), ang.sin().to(x.dtype)
        h = x.shape[-1] // 2
        a, b = x[..., :h], x[..., h:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1)


class SwiGLU(nn.Module):
    """``w_down(silu(w_gate x) * w_up x)`` (Shazeer, arXiv:2002.05202)."""

    def __init__(self, d_model, hidden):
        super().__init__()
        self.w_gate = Linear(d_model, hidden, bias=False)
        self.w_up = Linear(d_model, hidden, bias=False)
        self.w_down = Linear(hidden, d_model, bias=False)

    def forward(self, x):
        return self.w_down(F.silu(self.w_gate(x)) * self.w_up(x))


def _overlap_weights(n_cmp, n_slc, l, d, ls, device):
    """``W[i, j] = |[i d, i d + l) & [j ls, (j+1) ls)| / d``: how much of
    pooled token i falls in selection block j.  Identity when l = d = ls."""
    i = torch.arange(n_cmp, device=device, dtype=torch.float32)[:, None]
    j = torch.arange(n_slc, device=device, dtype=torch.float32)[None, :]
    lo = torch.maximum(i * d, j * ls)
    hi = torch.minimum(i * d + l, (j + 1) * ls)
    return (hi - lo).clamp(min=0) / d


def _stacked_padded(ws):
    """The weights stacked for one GEMM, with zero rows up to a multiple of 8
    outputs: the head split then moves 16-byte pieces of every output row
    (the padding columns come out 0, their gradient is written 0)."""
    pad = -sum(w.shape[0] for w in ws) % 8
    if pad:
        ws = tuple(ws) + (ws[0].new_zeros(pad, ws[0].shape[1]),)
    return torch.cat(ws, dim=0)


def _top_blocks(imp, k):
    """Top-k block indices per row, descending score then ascending index."""
    order = torch.sort(imp, dim=-1, descending=True, stable=True).indices
    return order[..., :k]


class NSAAttention(nn.Module):
    """NSA attention layer: shared query projection, per-branch key/value
    projections, learned compression poolers, per-head sigmoid gate over the
    three branches, output projection (nsa_model.py:130-195)."""

    def __init__(self, d_model, n_q_heads, n_kv_heads, block_size=16, n_selected_blocks=4, window=32,
                 attn_impl="ref", *, cmp_stride=None, sel_block=None, force_init=False, n_local=0, rope=None,
                 compressor="mean", cmp_hidden=None):
        super().__init__()
        assert n_q_heads % n_kv_heads == 0, "GQA needs n_q_heads divisible by n_kv_heads"
        assert attn_impl in ("ref", "fused"), "attn_impl must be 'ref' or 'fused'"
        assert compressor in ("mean", "mlp"), "compressor must be 'mean' (BlockCompressor) or 'mlp' (phi)"
        self.d_model = d_model
        self.Hq = n_q_heads
        self.Hkv = n_kv_heads
        self.G = n_q_heads // n_kv_heads
        self.dh = d_model // n_q_heads
        self.block_size = block_size
        self.cmp_stride = block_size if cmp_stride is None else cmp_stride
        self.sel_block = block_size if sel_block is None else sel_block
        self.force_init = bool(force_init)
        self.n_local = int(n_local)
        self.n_sel = n_selected_blocks
        self.window = window
        self.attn_impl = attn_impl
        self.rope = rope
        self.register_buffer("scale", torch.tensor(self.dh ** -0.5), persistent=False)

        kv_dim = self.Hkv * self.dh
        self.q_proj = Linear(d_model, self.Hq * self.dh, bias=False)
        self.k_cmp = Linear(d_model, kv_dim, bias=False)
        self.v_cmp = Linear(d_model, kv_dim, bias=False)
        self.k_slc = Linear(d_model, kv_dim, bias=False)
        self.v_slc = Linear(d_model, kv_dim, bias=False)
        self.k_win = Linear(d_model, kv_dim, bias=False)
        self.v_win = Linear(d_model, kv_dim, bias=False)
        self.compressor = compressor
        if compressor == "mlp":
            self.comp_k = MLPCompressor(block_size, self.dh, cmp_hidden)
            self.comp_v = MLPCompressor(block_size, self.dh, cmp_hidden)
        else:
            self.comp_k = BlockCompressor(block_size, self.dh)
            self.comp_v = BlockCompressor(block_size, self.dh)
        self.gate = Linear(d_model, self.Hq * 3, bias=True)
        self.out_proj = Linear(self.Hq * self.dh, d_model, bias=False)

    @property
    def aligned(self):
        """The reference's grid: one block size for all branches, nothing forced."""
        return (self.cmp_stride == self.block_size and self.sel_block == self.block_size
                and not self.force_init and self.n_local == 0)

    # -- shared pieces ------------------------------------------------------
    def _heads(self, y, n_heads):
        B, T, _ = y.shape
        return y.view(B, T, n_heads, self.dh).transpose(1, 2)

    def _n_cmp(self, T):
        l, d = self.block_size, self.cmp_stride
        return (T - l) // d + 1 if T >= l else 0

    def _pooled(self, kc, vc, n_cmp):
        """Learned pooled tokens of the spans ``[i d, i d + l)``, ``i < n_cmp``."""
        l, d = self.block_size, self.cmp_stride
        if self.compressor == "mlp" and self.attn_impl == "fused":
            T = (n_cmp - 1) * d + l
            return (self.comp_k.pool_sequence(kc[:, :, :T], d).to(kc.dtype),
                    self.comp_v.pool_sequence(vc[:, :, :T], d).to(vc.dtype))
        if self.attn_impl == "fused":
            # the learned mean on the HIP kernels (spans read in place); the
            # sequences are passed whole: their pooled tokens are the same n_cmp
            return self.comp_k.pool_sequence(kc, d), self.comp_v.pool_sequence(vc, d)
        if d == l:
            B = kc.shape[0]
            kb = kc[:, :, :n_cmp * l].reshape(B, self.Hkv, n_cmp, l, self.dh)
            vb = vc[:, :, :n_cmp * l].reshape(B, self.Hkv, n_cmp, l, self.dh)
        else:
            kb = kc[:, :, :(n_cmp - 1) * d + l].unfold(2, l, d).transpose(-1, -2)
            vb = vc[:, :, :(n_cmp - 1) * d + l].unfold(2, l, d).transpose(-1, -2)
        return self.comp_k(kb), self.comp_v(vb)

    def decode_cache(self, batch, capacity, dtype=None, device=None):
        """An ``NSADecodeCache`` for this layer: its geometry, and its own
        learned compressors pooling the compression caches (the prompt's
        spans and each span a decode step completes), so that a decode step
        is row t of ``forward`` (with the candidate blocks of t's whole
        selection block)."""
        import nsa_decode
        import nsa_hip_ops as ops
        p = next(self.parameters())
        geom = ops.NSAGeometry(self.block_size, self.cmp_stride, self.sel_block, self.n_sel, self.window,
                               self.force_init, self.n_local)

        def compress(k, v):
            kp, vp = self._pooled(k, v, self._n_cmp(k.shape[2]))
            return kp.to(k.dtype), vp.to(v.dtype)
        return nsa_decode.NSADecodeCache(batch, self.Hkv, self.dh, capacity, geom, dtype or p.dtype,
                                         device or p.device, compressor=compress)

    def _gate_logits(self, x):
        B, T, _ = x.shape
        return self.gate(x).view(B, T, self.Hq, 3).permute(0, 2, 1, 3)      # [B,Hq,T,3]

    def _stacked_weights(self):
        return (self.q_proj.weight, self.k_cmp.weight, self.v_cmp.weight, self.k_slc.weight, self.v_slc.weight,
                self.k_win.weight, self.v_win.weight, self.gate.weight)

    def _split_fused(self, x):
        """The fused path's inputs from the stacked projection of ``x`` in one
        head-split kernel: q, kc, vc, ks, vs, kw, vw head-major ([B, H, T, dh],
        q and the keys rotated when the model uses RoPE) and the gate logits
        [B, Hq, T, 3] with the gate's bias."""
        import nsa_hip_ops as ops
        y = _linear(x, _stacked_padded(self._stacked_weights()))
        r = self.rope is not None
        cos, sin = self.rope.tables(x.shape[1], y.device, y.dtype) if r else (None, None)
        kv = (self.Hkv, self.dh)
        segs = ((self.Hq, self.dh, r), (*kv, r), (*kv, False), (*kv, r), (*kv, False), (*kv, r), (*kv, False),
                (self.Hq, 3, False))
        return ops.split_heads(y, segs, cos, sin, bias=self.gate.bias, bias_seg=7)

    def _merge(self, out):
        B, _, T, _ = out.shape
        return self.out_proj(out.transpose(1, 2).reshape(B, T, self.Hq * self.dh))

    def _rot(self, y):
        return y if self.rope is None else self.rope(y)

    def forward(self, x, block_idx=None):
        if self.attn_impl == "fused":
            return self._forward_fused(x, block_idx)
        return self._forward_ref(x, block_idx)

    # -- dense torch definition (nsa_model.py:196-304) ------------------------
    def _block_choice(self, p_cmp, T, dev):
        """Selection scores from the compression probabilities (group sum,
        overlap map, causal mask, forcing) -> top-S block indices."""
        B, n = p_cmp.shape[0], p_cmp.shape[-1]
        ls = self.sel_block
        n_slc = T // ls
        imp = p_cmp.detach().float().view(B, self.Hkv, self.G, T, n).sum(dim=2)
        if not (self.cmp_stride == self.block_size == ls):
            imp = imp @ _overlap_weights(n, n_slc, self.block_size, self.cmp_stride, ls, dev)
        t = torch.arange(T, device=dev)
        j = torch.arange(n_slc, device=dev)
        valid = (j[None, :] + 1) * ls - 1 <= t[:, None]
        imp = imp.masked_fill(~valid, torch.finfo(imp.dtype).min)
        if self.force_init or self.n_local > 0:
            forced = torch.zeros(T, n_slc, dtype=torch.bool, device=dev)
            if self.force_init and n_slc > 0:
                forced[:, 0] = True
            for m in range(self.n_local):
                jl = t // ls - m
                ok = (jl >= 0) & (jl < n_slc)
                forced[t[ok], jl[ok]] = True
            imp = imp.masked_fill(forced, float("inf"))
        return _top_blocks(imp, min(self.n_sel, n_slc))

    def _forward_ref(self, x, block_idx=None):
        B, T, _ = x.shape
        l, d, ls = self.block_size, self.cmp_stride, self.sel_block
        n_cmp = self._n_cmp(T)
        n_slc = T // ls
        dev = x.device
        q = self._rot(self._heads(self.q_proj(x), self.Hq))
        kc = self._rot(self._heads(self.k_cmp(x), self.Hkv))
        vc = self._heads(self.v_cmp(x), self.Hkv)
        t = torch.arange(T, device=dev)

        o_cmp = q.new_zeros(q.shape)
        o_slc = q.new_zeros(q.shape)
        if n_cmp > 0:
            k_cmp, v_cmp = self._pooled(kc, vc, n_cmp)
            # pooled token i is visible once its whole span is in the past
            cmp_vis = torch.arange(n_cmp, device=dev) * d + l - 1 <= t[:, None]          # [T, n_cmp]
            s_cmp = _scores(q, expand_kv(k_cmp, self.G), self.scale)
            p_cmp = masked_softmax(s_cmp, cmp_vis.expand(B, self.Hq, T, n_cmp))
            o_cmp = p_cmp @ expand_kv(v_cmp, self.G)
            if n_slc > 0:
                if block_idx is None:
                    sel = self._block_choice(p_cmp, T, dev)                           # [B,Hkv,T,S]
                else:
                    sel = block_idx.to(device=dev, dtype=torch.long)
                self.last_block_idx = sel.to(torch.int32)
                hit = torch.zeros(B, self.Hkv, T, n_slc, dtype=torch.int32, device=dev)
                hit.scatter_add_(-1, sel.clamp(0, n_slc - 1), ((sel >= 0) & (sel < n_slc)).to(torch.int32))
                chosen = hit > 0
                blk_of_tok = (t // ls).clamp(max=n_slc - 1)
                sel_keep = chosen[..., blk_of_tok] & (t[None, :] <= t[:, None]) & (t < n_slc * ls)
                ks = expand_kv(self._rot(self._heads(self.k_slc(x), self.Hkv)), self.G)
                vs = expand_kv(self._heads(self.v_slc(x), self.Hkv), self.G)
                o_slc = masked_softmax(_scores(q, ks, self.scale), expand_kv(sel_keep, self.G)) @ vs

        kw = expand_kv(self._rot(self._heads(self.k_win(x), self.Hkv)), self.G)
        vw = expand_kv(self._heads(self.v_win(x), self.Hkv), self.G)
        win_keep = (t[None, :] <= t[:, None]) & (t[:, None] - t[None, :] < self.window)
        o_win = masked_softmax(_scores(q, kw, self.scale), win_keep.expand(B, self.Hq, T, T)) @ vw

        g = torch.sigmoid(self._gate_logits(x))
        out = g[..., 0:1] * o_cmp + g[..., 1:2] * o_slc + g[..., 2:3] * o_win
        return self._merge(out)

    # -- HIP kernels (nsa_model.py:306-370) -----------------------------------
    def _forward_fused(self, x, block_idx=None):
        import nsa_hip_ops as ops

        B, T, _ = x.shape
        n_cmp = self._n_cmp(T)
        q, kc, vc, ks, vs, kw, vw, gate_logits = self._split_fused(x)
        if n_cmp > 0:
            k_cmp, v_cmp = self._pooled(kc, vc, n_cmp)
        else:
            k_cmp = q.new_zeros(B, self.Hkv, 0, self.dh)
            v_cmp = q.new_zeros(B, self.Hkv, 0, self.dh)
        k_cmp, v_cmp, ks, vs, kw, vw, gate_logits = (y.to(q.dtype) for y in (k_cmp, v_cmp, ks, vs, kw, vw,
                                                                             gate_logits))
        geom = ops.NSAGeometry(self.block_size, self.cmp_stride, self.sel_block, self.n_sel, self.window,
                               self.force_init, self.n_local)
        if block_idx is not None:
            block_idx = block_idx.to(device=q.device, dtype=torch.int32)
        out, block_idx = ops.nsa_attention_layer(q, k_cmp.contiguous(), v_cmp.contiguous(), ks, vs, kw, vw,
                                                 gate_logits, geom, block_idx=block_idx, pooled=True)
        self.last_block_idx = block_idx
        return self._merge(out)


class FullAttention(nn.Module):
    """Dense causal GQA attention, the control arm (nsa_model.py:377-419): the
    same query / key / value / output projections as NSA without its three
    branches, compressors and gate.  ``impl='ref'`` materialises the full
    causal score matrix (as the reference does); ``impl='sdpa'`` runs the
    same function through ``scaled_dot_product_attention`` (flash kernels),
    the fair dense baseline at long sequences."""

    def __init__(self, d_model, n_q_heads, n_kv_heads, *, rope=None, impl="ref"):
        super().__init__()
        assert n_q_heads % n_kv_heads == 0, "GQA needs n_q_heads divisible by n_kv_heads"
        assert impl in ("ref", "sdpa"), "impl must be 'ref' or 'sdpa'"
        self.Hq = n_q_heads
        self.Hkv = n_kv_heads
        self.G = n_q_heads // n_kv_heads
        self.dh = d_model // n_q_heads
        self.rope = rope
        self.impl = impl
        self.register_buffer("scale", torch.tensor(self.dh ** -0.5), persistent=False)
        self.q_proj = Linear(d_model, self.Hq * self.dh, bias=False)
        self.k_proj = Linear(d_model, self.Hkv * self.dh, bias=False)
        self.v_proj = Linear(d_model, self.Hkv * self.dh, bias=False)
        self.out_proj = Linear(self.Hq * self.dh, d_model, bias=False)

    def _heads(self, y, n_heads):
        B, T, _ = y.shape
        return y.view(B, T, n_heads, self.dh).transpose(1, 2)

    def forward(self, x):
        B, T, _ = x.shape
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        if self.impl == "sdpa" and x.is_cuda:
            # the plumbing of NSAAttention's fused path: one GEMM over the
            # stacked weights (parameters kept separate), then one head-split
            # kernel (RoPE folded in) for q, k, v
            import nsa_hip_ops as ops
            y = _linear(x, _stacked_padded(ws))
            r = self.rope is not None
            cos, sin = self.rope.tables(T, y.device, y.dtype) if r else (None, None)
            q, k, v = ops.split_heads(y, ((self.Hq, self.dh, r), (self.Hkv, self.dh, r), (self.Hkv, self.dh, False)),
                                      cos, sin)
        else:
            if self.impl == "sdpa":
                yq, yk, yv = torch.split(F.linear(x, torch.cat(ws, dim=0)), [w.shape[0] for w in ws], dim=-1)
            else:
                yq, yk, yv = self.q_proj(x), self.k_proj(x), self.v_proj(x)
            q = self._heads(yq, self.Hq)
            k = self._heads(yk, self.Hkv)
            v = self._heads(yv, self.Hkv)
            if self.rope is not None:
                q, k = self.rope(q), self.rope(k)
        if self.impl == "sdpa":
            # fused kernels only (the unfused math fallback forms batched
            # products with transposed operands, avoided on this GPU), with
            # the KV heads shared by their query groups inside the kernel
            from torch.nn.attention import SDPBackend, sdpa_kernel
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                o = F.scaled_dot_product_attention(q.contiguous(), k.contiguous(), v.contiguous(), is_causal=True,
                                                   enable_gqa=self.G > 1)
        else:
            k, v = expand_kv(k, self.G), expand_kv(v, self.G)
            causal = torch.ones(T, T, dtype=torch.bool, device=x.device).tril()
            o = masked_softmax(_scores(q, k, self.scale), causal[None, None]) @ v
        return self.out_proj(o.transpose(1, 2).reshape(B, T, self.Hq * self.dh))


def make_attention(attn_type, d_model, n_q_heads, n_kv_heads, **nsa_kw):
    """``'nsa'`` -> NSAAttention(**nsa_kw); ``'full'`` -> FullAttention (the NSA
    keywords do not apply to it), as nsa_model.py:426-432."""
    if attn_type == "nsa":
        return NSAAttention(d_model, n_q_heads, n_kv_heads, **nsa_kw)
    if attn_type == "full":
        return FullAttention(d_model, n_q_heads, n_kv_heads, rope=nsa_kw.get("rope"),
                             impl=nsa_kw.get("dense_impl", "ref"))
    raise ValueError(f"unknown attn_type {attn_type!r} (expected 'nsa' or 'full')")


_NSA_ONLY = ("block_size", "n_selected_blocks", "window", "attn_impl", "cmp_stride", "sel_block", "force_init",
             "n_local", "compressor", "cmp_hidden")


class Block(nn.Module):
    """Pre-norm residual block: ``x + attn(norm1(x))``, then
    ``x + ffn(norm2(x))`` (nsa_model.py:435-452).  Defaults are the
    reference's (LayerNorm, GELU MLP of ``ffn_mult * d_model``); ``norm='rms'``
    and ``ffn='swiglu'`` give the Llama-style variant."""

    def __init__(self, d_model, n_q_heads, n_kv_heads, ffn_mult=4, attn_type="nsa", *, norm="layer",
                 ffn="gelu", ffn_hidden=None, **nsa_kw):
        super().__init__()
        if attn_type == "full":
            nsa_kw = {k: v for k, v in nsa_kw.items() if k not in _NSA_ONLY}
        else:
            nsa_kw = {k: v for k, v in nsa_kw.items() if k != "dense_impl"}
        self.ln1 = _norm(norm, d_model)
        self.attn = make_attention(attn_type, d_model, n_q_heads, n_kv_heads, **nsa_kw)
        self.ln2 = _norm(norm, d_model)
        hidden = ffn_mult * d_model if ffn_hidden is None else ffn_hidden
        if ffn == "swiglu":
            self.ffn = SwiGLU(d_model, hidden)
        else:
            assert ffn == "gelu", "ffn must be 'gelu' or 'swiglu'"
            self.ffn = nn.Sequential(Linear(d_model, hidden), nn.GELU(), Linear(hidden, d_model))

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.ffn(self.ln2(x))


def _norm(kind, d_model):
    assert kind in ("layer", "rms"), "norm must be 'layer' or 'rms'"
    return nn.LayerNorm(d_model) if kind == "layer" else nn.RMSNorm(d_model)


class NSATransformer(nn.Module):
    """Decoder-only language model with NSA (or dense) attention in every
    block: token embedding (+ learned positions unless ``pos='rope'``), the
    blocks, final norm, LM head tied to the embedding (nsa_model.py:455-511).
    ``forward(idx, targets=None) -> (logits, loss)``; ``grad_checkpoint``
    recomputes each block in the backward."""

    def __init__(self, vocab_size, d_model=512, n_layers=8, n_q_heads=8, n_kv_heads=2, max_seq_len=256,
                 ffn_mult=4, block_size=16, n_selected_blocks=4, window=32, attn_type="nsa", attn_impl="ref", *,
                 norm="layer", ffn="gelu", ffn_hidden=None, pos="learned", rope_base=10000.0, tie_embeddings=True,
                 dense_impl="ref", cmp_stride=None, sel_block=None, force_init=False, n_local=0, compressor="mean",
                 cmp_hidden=None):
        super().__init__()
        assert pos in ("learned", "rope"), "pos must be 'learned' or 'rope'"
        self.max_seq_len = max_seq_len
        self.attn_type = attn_type
        self.attn_impl = attn_impl
        self.grad_checkpoint = False
        self.tok_emb = nn.Embedding(vocab_size, d_model)
        rope = Rotary(d_model // n_q_heads, rope_base) if pos == "rope" else None
        if pos == "learned":
            self.pos_emb = nn.Embedding(max_seq_len, d_model)
        kw = dict(attn_impl=attn_impl, block_size=block_size, n_selected_blocks=n_selected_blocks, window=window,
                  cmp_stride=cmp_stride, sel_block=sel_block, force_init=force_init, n_local=n_local, rope=rope,
                  dense_impl=dense_impl, compressor=compressor, cmp_hidden=cmp_hidden)
        self.blocks = nn.ModuleList([Block(d_model, n_q_heads, n_kv_heads, ffn_mult=ffn_mult, attn_type=attn_type,
                                           norm=norm, ffn=ffn, ffn_hidden=ffn_hidden, **kw)
                                     for _ in range(n_layers)])
        self.ln_f = _norm(norm, d_model)
        self.lm_head = Linear(d_model, vocab_size, bias=False)
        if tie_embeddings:
            self.lm_head.weight = self.tok_emb.weight
        self.apply(self._init)

    @staticmethod
    def _init(m):
        """N(0, 0.02) for every linear and embedding weight, zero biases
        (nsa_model.py:477-484)."""
        if isinstance(m, (nn.Linear, nn.Embedding)):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
        if isinstance(m, nn.Linear) and m.bias is not None:
            nn.init.zeros_(m.bias)

    def forward(self, idx, targets=None):
        B, T = idx.shape
        assert T <= self.max_seq_len
        x = self.tok_emb(idx)
        if hasattr(self, "pos_emb"):
            x = x + self.pos_emb(torch.arange(T, device=idx.device))[None]
        for blk in self.blocks:
            if self.grad_checkpoint and self.training:
                x = torch.utils.checkpoint.checkpoint(blk, x, use_reentrant=False)
            else:
                x = blk(x)
        logits = self.lm_head(self.ln_f(x))
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1))
        return logits, loss

    def num_params(self):
        """The reference's parameter count (nsa_model.py:508-511): the unique
        parameters minus the LM head matrix (with tied weights that leaves
        the embedding out as well)."""
        return sum(p.numel() for p in self.parameters()) - self.lm_head.weight.numel()


# parameter-name keyword -> branch label, first match wins (nsa_model.py:524-537)
_BRANCH_RULES = [
    ("attn.q_proj", "q_proj (shared)"),
    ("attn.k_cmp", "compression"), ("attn.v_cmp", "compression"),
    ("attn.comp_k", "compression"), ("attn.comp_v", "compression"),
    ("attn.k_slc", "selection"), ("attn.v_slc", "selection"),
    ("attn.k_win", "window"), ("attn.v_win", "window"),
    ("attn.gate", "gate"),
    ("attn.out_proj", "out_proj"),
    ("ffn", "ffn"),
    ("tok_emb", "embed"), ("pos_emb", "embed"),
    ("ln", "layernorm"),
]

# branches that must receive gradient (nsa_model.py:540)
REQUIRED_BRANCHES = ["q_proj (shared)", "compression", "selection", "window", "gate"]


def branch_of(param_name):
    """Branch label of a parameter name (nsa_model.py:543-547)."""
    return next((label for key, label in _BRANCH_RULES if key in param_name), "other")


def param_groups(model):
    """``{branch label: [(name, param), ...]}`` (nsa_model.py:550-556)."""
    groups = {}
    for name, p in model.named_parameters():
        groups.setdefault(branch_of(name), []).append((name, p))
    return groups
