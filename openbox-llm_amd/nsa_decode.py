"""Decode / KV-cache path of NSA on MI355X: one new query per sequence.

The reference runs whole sequences only (NSAAttention.forward,
nsa_model.py:196-304).  A decode step here computes that function's row
``t = len - 1`` for every sequence of a batch from per-layer caches, with
the candidate blocks ``0 .. t // sel_block`` (the row of a prefill whose
length reaches the end of t's selection block, so the step does not depend on
how long the sequence will grow):

* ``NSADecodeCache`` holds one layer's caches -- the six branch K/V caches
  ``[B, Hkv, capacity, D]``, the pooled compression caches and the lengths
  (int32, on the device) -- and runs ``prefill`` / ``append`` / ``attend``.
* ``attend`` is ``nsa_decode_fwd``: split-K compression and window partials,
  single-query importance + top-n (ties to the lower block), split-K over
  the picked blocks, then the gated merge: five launches (four when the
  pooled sequence fits two token-sum chunks, up to 2048 pooled tokens), no
  host sync.
* ``append`` is ``nsa_decode_append``: the new rows go to position ``len``
  and a pooled token is written when the new length completes a span, bit
  for bit what ``block_mean_pool`` (``nsa_pool_fwd``) gives over the whole
  sequence (the kernel-level NSA, nsa_fused_kernel.py:549-554).
* A model layer pools with learned compressors instead (BlockCompressor,
  nsa_model.py:100-123, or the MLP phi): a cache built with ``compressor``
  (``NSAAttention.decode_cache`` passes the layer's own) pools the prompt's
  spans with it and, after every append, the span the new length completes.

Lengths live on the device, so a generation loop of ``append`` + ``attend``
never waits for the host.
"""

import torch

import nsa_hip_ops as _ops
from nsa_hip_ops import NSAGeometry  # noqa: F401  (public)

decode_fwd = _ops.decode_fwd
decode_append = _ops.decode_append


class NSADecodeCache:
    """Caches of one NSA attention layer for ``batch`` sequences of up to
    ``capacity`` tokens (``n_kv_heads`` x ``head_dim``, ``dtype``)."""

    def __init__(self, batch, n_kv_heads, head_dim, capacity, geom: NSAGeometry, dtype=torch.bfloat16,
                 device="cuda", compressor=None):
        """``compressor`` (optional): ``(k, v) -> (k_pooled, v_pooled)``, the
        pooled tokens ``[B, Hkv, (T - l) // d + 1, D]`` of the spans ``[i d,
        i d + l)`` of ``k, v [B, Hkv, T, D]``; without it the caches hold the
        plain span means."""
        self.geom = geom
        self.compressor = compressor
        shape = (batch, n_kv_heads, capacity, head_dim)
        self.kc, self.vc, self.ks, self.vs, self.kw, self.vw = [
            torch.zeros(shape, device=device, dtype=dtype) for _ in range(6)]
        ncap = max(1, _ops.n_cmp_tokens(capacity, geom.cmp_block, geom.cmp_stride))
        self.k_cmp = torch.zeros(batch, n_kv_heads, ncap, head_dim, device=device, dtype=dtype)
        self.v_cmp = torch.zeros_like(self.k_cmp)
        self.lens = torch.zeros(batch, device=device, dtype=torch.int32)
        self._ws = {}

    @property
    def capacity(self):
        return self.kc.shape[2]

    def caches(self):
        return (self.kc, self.vc, self.ks, self.vs, self.kw, self.vw)

    def prefill(self, kc, vc, ks, vs, kw, vw, lens=None):
        """Load a prompt's branch keys / values ``[B, Hkv, T, D]`` (T <=
        capacity); ``lens`` (int, or one per sequence, each <= T) says how
        many of the T rows each sequence holds (default T)."""
        T = kc.shape[2]
        assert T <= self.capacity, "prompt longer than the cache"
        for dst, src in zip(self.caches(), (kc, vc, ks, vs, kw, vw)):
            assert src.shape == dst.shape[:2] + (T, dst.shape[3]), "prompt K/V must be [B, Hkv, T, D]"
            dst[:, :, :T].copy_(src)
        n = _ops.n_cmp_tokens(T, self.geom.cmp_block, self.geom.cmp_stride)
        if n > 0:
            # pooled tokens whose span runs past a sequence's length are
            # rewritten by append before they become visible
            kc_t, vc_t = self.kc[:, :, :T], self.vc[:, :, :T]
            if self.compressor is not None:
                kp, vp = self.compressor(kc_t, vc_t)
            else:
                kp = _ops.pool_fwd(kc_t, self.geom.cmp_block, self.geom.cmp_stride)
                vp = _ops.pool_fwd(vc_t, self.geom.cmp_block, self.geom.cmp_stride)
            self.k_cmp[:, :, :n].copy_(kp)
            self.v_cmp[:, :, :n].copy_(vp)
        if lens is None:
            self.lens.fill_(T)
        else:
            lens = torch.as_tensor(lens, dtype=torch.int32).to(self.lens.device)
            assert int(lens.max()) <= T and int(lens.min()) >= 0
            self.lens.copy_(lens.expand_as(self.lens))

    def append(self, kc, vc, ks, vs, kw, vw):
        """Append one token per sequence (rows ``[B, Hkv, D]``)."""
        self.lens = _ops.decode_append(*self.caches(), self.k_cmp, self.v_cmp, (kc, vc, ks, vs, kw, vw),
                                       self.lens, self.geom)
        if self.compressor is not None:
            self._recompress_last_span()

    def _recompress_last_span(self):
        """With a learned compressor: pool the span each sequence's new length
        completes (span (len - l) / d, when it divides) with it, over the
        mean the append kernel wrote; sequences whose length completes no span
        keep their pooled tokens.  All on the device (no host sync)."""
        l, d = self.geom.cmp_block, self.geom.cmp_stride
        B = self.kc.shape[0]
        L = self.lens.long()
        i = torch.clamp((L - l) // d, min=0)
        done = (L >= l) & ((L - l) % d == 0)
        pos = torch.clamp(i[:, None] * d + torch.arange(l, device=L.device)[None, :], max=self.capacity - 1)
        b = torch.arange(B, device=L.device)
        ks = self.kc[b[:, None], :, pos].permute(0, 2, 1, 3)          # [B, Hkv, l, D]
        vs = self.vc[b[:, None], :, pos].permute(0, 2, 1, 3)
        kp, vp = self.compressor(ks.contiguous(), vs.contiguous())      # [B, Hkv, 1, D]
        for cache, new in ((self.k_cmp, kp), (self.v_cmp, vp)):
            old = cache[b, :, i]                                        # [B, Hkv, D]
            cache[b, :, i] = torch.where(done[:, None, None], new[:, :, 0].to(cache.dtype), old)

    def _workspace(self, Hq, D):
        if Hq not in self._ws:
            B, Hkv, Tcap, _ = self.kc.shape
            nbytes = _ops.decode_workspace_bytes(B, Hq, Hkv, D, Tcap, self.k_cmp.shape[2], self.geom)
            self._ws[Hq] = torch.empty(nbytes, device=self.kc.device, dtype=torch.uint8)
        return self._ws[Hq]

    def attend(self, q, gate, **kw):
        """NSA output of the newest token of every sequence: ``q [B, Hq, D]``,
        ``gate [B, Hq, 3]`` logits -> ``(out [B, Hq, D], block_idx)`` (see
        ``nsa_hip_ops.decode_fwd`` for the optional extras)."""
        return _ops.decode_fwd(q, self.k_cmp, self.v_cmp, self.ks, self.vs, self.kw, self.vw, gate, self.lens,
                               self.geom, workspace=self._workspace(q.shape[1], q.shape[2]), **kw)

    def step(self, q, gate, new_rows, **kw):
        """``append(*new_rows)`` then ``attend(q, gate)``."""
        self.append(*new_rows)
        return self.attend(q, gate, **kw)
