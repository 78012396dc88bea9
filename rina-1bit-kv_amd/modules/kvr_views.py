"""Reference-compatible per-layer objects over a layer's TileKVCache.

The reference hook keeps one WindowBuffer and one RetrievalIndex per layer
(modules/kvr_hook.py:43-47) and its scripts read them directly, e.g.
`hook.retrievals[li].compute_all_scores(q)`, `ret.n_stored`, `ret._deq_k(h)`,
`ret._rotary(k, idx)` (scripts/evaluation/_diag_rank.py:59-83), or set
`.chunk_size` / `.attractors` / `.n_attractors` / `.top_per_basin`
(scripts/evaluation/_test_int4.py:33-36, kvr_attractor_sweep.py:108).  Here one
TileKVCache holds both, so KVRHook.windows[li] and KVRHook.retrievals[li] are views
of it for one sequence b (0 by default):

  CacheWindowView    : k, v (the window's tokens in order, (n, n_kv, d), a copy), n,
                       pos (tokens that entered the window so far), cap (ring slots),
                       attention(q) (exact window attention on the HIP kernel),
                       append(k, v) (B == 1 caches).
  CacheRetrievalView : a RetrievalIndex over the cache's tile store (n_stored =
                       evicted tokens, all encoded; the window's tokens are not in it):
                       compute_all_scores, compute_chunk_scores, retrieve_topk,
                       retrieve, _deq_k, _rotary, with the model's RoPE tables.  The
                       k-means attributes are accepted and have no effect, as in
                       RetrievalIndex.  The store is filled by the hook only
                       (calibrate / append / batch_append raise).
"""
from __future__ import annotations

import torch

from . import _hip
from .kvr_retrieval import RetrievalIndex


class CacheWindowView:
    def __init__(self, hook, li, b=0):
        self._hook, self._li, self._b = hook, li, b
        self.n_kv = hook.n_kv
        self.d_head = hook.d_head

    @property
    def cache(self):
        c = self._hook.caches[self._li]
        if c is None:
            raise RuntimeError("the hook has no cache for this layer yet (call prefill first)")
        return c

    @property
    def n(self):
        return self.cache.n

    @property
    def pos(self):
        c = self.cache
        return c.n_tiles * c.T + c.n

    @property
    def cap(self):
        return self.cache.cap

    @property
    def k(self):
        return self.cache.window_tokens()[0][self._b].permute(1, 0, 2)

    @property
    def v(self):
        return self.cache.window_tokens()[1][self._b].permute(1, 0, 2)

    @torch.no_grad()
    def append(self, k_post_rope, v):
        c = self.cache
        if c.B != 1:
            raise RuntimeError("append through the view needs a batch-1 cache (use TileKVCache.append)")
        c.append(k_post_rope.reshape(1, c.Hkv, 128), v.reshape(1, c.Hkv, 128))

    @torch.no_grad()
    def attention(self, q_post_rope, n_q=None, scale=None):
        """Exact softmax attention of q (n_q, d) over the window's tokens; float32 (n_q, d)
        like the reference (kvr_window.py:43-69)."""
        c = self.cache
        n_q = n_q or q_post_rope.shape[0]
        q = q_post_rope.reshape(1, n_q, self.d_head)
        if q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            q = q.float()
        if scale is not None and abs(scale - self.d_head ** 0.5) > 1e-12 * scale:
            q = q.float() * (self.d_head ** 0.5 / scale)  # the kernel divides by sqrt(d)
        if c.n == 0:
            return torch.zeros((n_q, self.d_head), device=q.device, dtype=torch.float32)
        b = self._b
        out = _hip.decode_attn(q.contiguous(), c.win_k[b:b + 1], c.win_v[b:b + 1], c.n, None, None, None, None,
                               None, c.T, _hip.NONE, out_dtype=torch.float32, win_start=c.start, win_cap=c.cap)
        return out[0]


class CacheRetrievalView(RetrievalIndex):
    # pylint: disable=super-init-not-called
    def __init__(self, hook, li, b=0):
        self._hook, self._li, self._b = hook, li, b
        self.n_kv = hook.n_kv
        self.d_head = hook.d_head
        self.kv_dim = self.n_kv * self.d_head
        self.top_k = hook.top_k
        self.chunk_size = hook.chunk_size  # accepted, no effect (tiles of T tokens are used)
        self.tile = hook.tile
        self.transform = hook.transform
        self.device = hook.device
        self.attractors = None
        self.labels = None
        self.n_attractors = 128
        self.top_per_basin = 16
        self._calibrated = True
        self._tables = (0, None, None)

    @property
    def cache(self):
        c = self._hook.caches[self._li]
        if c is None:
            raise RuntimeError("the hook has no cache for this layer yet (call prefill first)")
        return c

    def _rows(self, t):
        b, h = self._b, self.n_kv
        return t[b * h:(b + 1) * h]

    kbits = property(lambda self: self._rows(self.cache.kbits))
    kscale = property(lambda self: self._rows(self.cache.kscale))
    vbits = property(lambda self: self._rows(self.cache.vbits))
    vscale = property(lambda self: self._rows(self.cache.vscale))
    n_tiles = property(lambda self: self.cache.n_tiles)

    @property
    def tail_k(self):  # the cache's unencoded tokens live in its window, not here
        return torch.zeros((0, self.n_kv, self.d_head), dtype=torch.float32, device=self.device)

    tail_v = tail_k

    def _rope_tables(self, n):
        """cos / sin (n, d) fp32 of absolute positions 0..n-1 from the model's rotary embedding."""
        have, cos, sin = self._tables
        if have < n:
            rot = self._hook.model.model.rotary_emb
            ref = torch.zeros(1, device=self.device, dtype=torch.float32)
            pos = torch.arange(n, device=self.device)[None]
            c, s = rot(ref, position_ids=pos)
            cos, sin = c[0].float(), s[0].float()
            self._tables = (n, cos, sin)
        return cos[:n], sin[:n]

    @property
    def cos(self):
        return self._rope_tables(max(1, self.n_stored))[0]

    @property
    def sin(self):
        return self._rope_tables(max(1, self.n_stored))[1]

    def set_rotary_tables(self, cos, sin):
        raise RuntimeError("the hook's stores use the model's rotary embedding")

    def calibrate(self, *a, **k):
        raise RuntimeError("the hook fills its stores itself (prefill / decode)")

    append = batch_append = calibrate
