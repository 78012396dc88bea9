"""RetrievalIndex -- the compressed store of evicted tokens (drop-in for the reference's
modules/kvr_retrieval.py:40-412), backed by the 1-bit tile codec on gfx950.

Reference behaviour kept: constructor and method names, `calibrate` before `append`
(RuntimeError otherwise, :164-165), `batch_append` REPLACES the store (:193-194), RoPE
convention of the rotary tables (:27-37, tables set by `set_rotary_tables`), GQA-mean
query and cosine scoring (:270, :284-286), chunk(=tile)-level top-k with
k = min(max(1, top_k // T), n_tiles) (:378), exclusion of [exclude_start, exclude_end)
converted to tiles as :373-377, empty returns (:323-326), and the return convention of
retrieve_topk: (K_post float32 (m, n_kv, d), V float16 (m, n_kv, d)) (:411-412).

Codec differences (the point of the rebuild): tokens are stored post-RoPE, rotated along
head_dim (Hadamard-128 or DCT-II-128) and sigma-delta coded to 1 bit in tiles of T tokens
with one fp16 scale per tile for K and for V; there is no global calibration (`calibrate`
only resets the store), no W-predicted V and no k-means attractors (`build_attractors` is a
no-op, `attractors` stays None).  Appended tokens wait in an exact staging tail until T of
them complete a tile; retrieve_topk returns the selected tiles' tokens followed by the tail.
"""
from __future__ import annotations

import torch

from . import _hip


def _rotate_half(x):
    d2 = x.shape[-1] // 2
    return torch.cat([-x[..., d2:], x[..., :d2]], dim=-1)


def _apply_rotary(x, cos, sin):
    """x * cos + rotate_half(x) * sin (kvr_retrieval.py:32-33)."""
    return x * cos[:x.shape[0]] + _rotate_half(x) * sin[:x.shape[0]]


def _reverse_rotary(x, cos, sin):
    """x * cos - rotate_half(x) * sin (kvr_retrieval.py:36-37)."""
    return x * cos[:x.shape[0]] - _rotate_half(x) * sin[:x.shape[0]]


class RetrievalIndex:
    def __init__(self, n_kv, d_head, top_k=128, device='cuda', chunk_size=8, tile=64, transform='hadamard'):
        if d_head != 128:
            raise ValueError("the HIP kernels are built for head_dim 128")
        self.n_kv = n_kv
        self.d_head = d_head
        self.kv_dim = n_kv * d_head
        self.top_k = top_k
        self.chunk_size = chunk_size          # reference attribute; tiles of `tile` tokens are used
        self.tile = tile
        self.transform = _hip.TRANSFORMS[transform] if isinstance(transform, str) else transform
        self.device = device
        self.cos = None
        self.sin = None
        self.attractors = None
        self.labels = None
        self.n_attractors = 128
        self.top_per_basin = 16
        self._calibrated = False
        self._reset_store()

    # ------------------------------------------------------------------ state
    def _reset_store(self, cap_tiles=16):
        self.kbits, self.kscale = _hip.alloc_store(self.n_kv, cap_tiles, self.tile, self.device)
        self.vbits, self.vscale = _hip.alloc_store(self.n_kv, cap_tiles, self.tile, self.device)
        self.n_tiles = 0
        self.tail_k = torch.zeros((0, self.n_kv, self.d_head), dtype=torch.float32, device=self.device)
        self.tail_v = torch.zeros_like(self.tail_k)

    @property
    def n_stored(self):
        return self.n_tiles * self.tile + self.tail_k.shape[0]

    def _ensure_tiles(self, need):
        cap = self.kbits.shape[1]
        if need <= cap:
            return
        new_cap = max(need, 2 * cap)
        for name in ("kbits", "vbits", "kscale", "vscale"):
            old = getattr(self, name)
            new = torch.zeros((old.shape[0], new_cap) + tuple(old.shape[2:]), dtype=old.dtype, device=old.device)
            new[:, :cap] = old
            setattr(self, name, new)

    def set_rotary_tables(self, cos, sin):
        self.cos = cos
        self.sin = sin

    def _rotary(self, k_pre, positions):
        """Post-RoPE keys at absolute positions (kvr_retrieval.py:136-141)."""
        if self.cos is None:
            return k_pre.float()
        c = self.cos[positions].to(torch.float32)[:, None, :]
        s = self.sin[positions].to(torch.float32)[:, None, :]
        k = k_pre.float()
        return k * c + _rotate_half(k) * s

    def _flush_tiles(self):
        """Encode every complete tile of the tail into the store."""
        m = self.tail_k.shape[0] // self.tile
        if m == 0:
            return
        n = m * self.tile
        self._ensure_tiles(self.n_tiles + m)
        k = self.tail_k[:n].permute(1, 0, 2).unsqueeze(0)  # [1, n_kv, n, d] strided
        v = self.tail_v[:n].permute(1, 0, 2).unsqueeze(0)
        _hip.encode_tiles(k, self.tile, self.transform, bits=self.kbits, scales=self.kscale, tile_offset=self.n_tiles)
        _hip.encode_tiles(v, self.tile, self.transform, bits=self.vbits, scales=self.vscale, tile_offset=self.n_tiles)
        self.n_tiles += m
        self.tail_k = self.tail_k[n:].clone()
        self.tail_v = self.tail_v[n:].clone()

    # ------------------------------------------------------------------ building
    @torch.no_grad()
    def calibrate(self, k_pre_sample, v_sample=None):
        """Resets the store (the 1-bit codec needs no global calibration; kvr_retrieval.py:95-122)."""
        self._reset_store()
        self._calibrated = True

    @torch.no_grad()
    def append(self, k_pre_rope, v=None):
        """One token (n_kv, d), stored at position n_stored (kvr_retrieval.py:162-185)."""
        if not self._calibrated:
            raise RuntimeError("Call calibrate() first")
        pos = torch.tensor([self.n_stored], device=k_pre_rope.device)
        k = self._rotary(k_pre_rope.reshape(1, self.n_kv, self.d_head), pos)
        vv = torch.zeros_like(k) if v is None else v.reshape(1, self.n_kv, self.d_head).float()
        self.tail_k = torch.cat([self.tail_k, k])
        self.tail_v = torch.cat([self.tail_v, vv])
        self._flush_tiles()

    @torch.no_grad()
    def batch_append(self, k_pre_all, v_all):
        """Replaces the store with tokens 0..n-1 (kvr_retrieval.py:187-207)."""
        n = k_pre_all.shape[0]
        self._reset_store(cap_tiles=max(16, n // self.tile + 1))
        self._calibrated = True
        pos = torch.arange(n, device=k_pre_all.device)
        self.tail_k = self._rotary(k_pre_all, pos).contiguous()
        self.tail_v = v_all.float().contiguous()
        self._flush_tiles()

    # ------------------------------------------------------------------ files
    def save_store(self, f):
        """Write the store (tiles and the exact staging tail, as the window section with
        W = 0, fp32) to a store file (include/kvr_store.h).  No reference counterpart: the
        reference rebuilds its store on reset (kvr_retrieval.py:150-160)."""
        from . import kvr_store
        nt, tail = self.n_tiles, self.tail_k.shape[0]
        desc = kvr_store.new_desc(T=self.tile, transform=self.transform, n_layers=1, B=1, Hkv=self.n_kv,
                                  n_tiles=nt, W=0, win_len=tail, win_dtype=_hip.FP32, counts=False,
                                  user=(int(self._calibrated), 0, 0, 0))
        layer = {kvr_store.SEC_KBITS: self.kbits[:, :nt], kvr_store.SEC_VBITS: self.vbits[:, :nt],
                 kvr_store.SEC_KSCALE: self.kscale[:, :nt], kvr_store.SEC_VSCALE: self.vscale[:, :nt],
                 kvr_store.SEC_WIN_K: self.tail_k.permute(1, 0, 2).unsqueeze(0),
                 kvr_store.SEC_WIN_V: self.tail_v.permute(1, 0, 2).unsqueeze(0)}
        return kvr_store.write_layers(f, desc, [layer])

    @torch.no_grad()
    def load_store(self, f):
        """Replace the store with a store file's first layer (tiles + tail); the file must
        match this index's KV heads, tile size and transform."""
        from . import kvr_store
        desc, layers = kvr_store.read_layers(f)
        if (desc.B, desc.Hkv, desc.T, desc.transform) != (1, self.n_kv, self.tile, self.transform):
            raise ValueError(f"store {desc} does not match this index (n_kv={self.n_kv}, tile={self.tile}, "
                             f"transform={self.transform})")
        layer, nt = layers[0], int(desc.n_tiles)
        self._reset_store(cap_tiles=max(16, nt + 1))
        if nt:
            for sec, name in ((kvr_store.SEC_KBITS, "kbits"), (kvr_store.SEC_VBITS, "vbits"),
                              (kvr_store.SEC_KSCALE, "kscale"), (kvr_store.SEC_VSCALE, "vscale")):
                getattr(self, name)[:, :nt] = torch.from_numpy(layer[sec].copy())
        self.n_tiles = nt
        if desc.flags & kvr_store.HAS_WINDOW and desc.win_len:
            wdt = _hip._TORCH_DT[desc.win_dtype]
            self.tail_k, self.tail_v = (
                torch.from_numpy(layer[s].copy()).view(wdt)[0].permute(1, 0, 2).float().contiguous().to(self.device)
                for s in (kvr_store.SEC_WIN_K, kvr_store.SEC_WIN_V))
            self._flush_tiles()  # a tail of T or more tokens (W > 0 stores) goes to the tiles
        self._calibrated = True
        return desc

    def build_attractors(self):
        """k-means attractor basins are not part of the tile codec: no-op."""
        return None

    # ------------------------------------------------------------------ scoring
    def _qbar(self, q_post_rope, n_q):
        q = q_post_rope.reshape(1, n_q, self.d_head).float().contiguous()
        qbar, _ = _hip.query_prep(q, self.n_kv, self.transform, want_q_rot=False)
        return q, qbar

    @torch.no_grad()
    def compute_chunk_scores(self, q_post_rope):
        """Tile scores (n_tiles, n_kv): cosine of the rotated GQA-mean query with each tile's
        column sums (the chunk-mean cosine of kvr_retrieval.py:291-315)."""
        n_q = q_post_rope.shape[0]
        if self.n_tiles == 0:
            return torch.empty((0, self.n_kv), device=self.device)
        _, qbar = self._qbar(q_post_rope, n_q)
        return _hip.score_tiles(qbar, self.kbits, self.n_tiles, self.tile).t()

    def _tokens(self, bits, scales, idx):
        """Decoded tokens of tiles idx [n_kv, k]: [k*T, n_kv, d] fp32 (original domain)."""
        out = _hip.gather_tiles(bits, scales, idx, self.tile, self.transform)  # [n_kv, k*T, d]
        return out.permute(1, 0, 2)

    def _all_keys(self):
        """Every stored key, decoded, post-RoPE, in position order: (n_stored, n_kv, d) fp32."""
        keys = [self.tail_k]
        if self.n_tiles:
            idx = torch.arange(self.n_tiles, device=self.device, dtype=torch.int32).repeat(self.n_kv, 1)
            keys.insert(0, self._tokens(self.kbits, self.kscale, idx))
        return torch.cat(keys)

    @torch.no_grad()
    def _deq_k(self, kvh):
        """Decoded keys of KV head kvh as pre-RoPE fp32 (n_stored, d) (kvr_retrieval.py:125-129).
        The store holds post-RoPE keys, so they are rotated back: _rotary(_deq_k(h), positions)
        gives the decoded post-RoPE keys, the pattern of scripts/evaluation/_diag_rank.py:76-77."""
        k = self._all_keys()[:, kvh]
        if self.cos is None:
            return k
        n = k.shape[0]
        return _reverse_rotary(k, self.cos[:n].float(), self.sin[:n].float())

    @torch.no_grad()
    def compute_all_scores(self, q_post_rope):
        """Token-level cosine scores (n_stored, n_kv) on the decoded tokens (kvr_retrieval.py:265-289)."""
        n_q = q_post_rope.shape[0]
        g = n_q // self.n_kv
        q_avg = q_post_rope.float().view(self.n_kv, g, self.d_head).mean(dim=1)
        k = self._all_keys()
        qn = q_avg / (q_avg.norm(dim=-1, keepdim=True) + 1e-8)
        kn = k / (k.norm(dim=-1, keepdim=True) + 1e-8)
        scores = torch.einsum('hd,thd->th', qn, kn)
        return torch.where(torch.isnan(scores), torch.full_like(scores, float('-inf')), scores)

    # ------------------------------------------------------------------ retrieval
    @torch.no_grad()
    def retrieve_topk(self, q_post_rope, n_q=None, exclude_start=0, exclude_end=0):
        """Top-k tiles per KV head -> (K_post float32 (m, n_kv, d), V float16 (m, n_kv, d))."""
        n_q = n_q or q_post_rope.shape[0]
        d = self.d_head
        nr = self.n_stored
        empty = (torch.zeros(0, self.n_kv, d, device=self.device, dtype=torch.float16),
                 torch.zeros(0, self.n_kv, d, device=self.device, dtype=torch.float16))
        if nr == 0 or exclude_start >= nr:
            return empty
        if exclude_start <= 0 and exclude_end >= nr:
            return empty
        parts_k, parts_v = [], []
        if self.n_tiles:
            T = self.tile
            lo = exclude_start // T
            hi = min((exclude_end + T - 1) // T, self.n_tiles)
            if lo >= hi:
                lo = hi = 0
            k = min(max(1, self.top_k // T), self.n_tiles)
            _, qbar = self._qbar(q_post_rope, n_q)
            ex_lo = torch.full((self.n_kv,), lo, dtype=torch.int32, device=self.device)
            ex_hi = torch.full((self.n_kv,), hi, dtype=torch.int32, device=self.device)
            scores = _hip.score_tiles(qbar, self.kbits, self.n_tiles, T, excl_lo=ex_lo, excl_hi=ex_hi)
            idx = _hip.topk_tiles(scores, k)
            self.last_idx = idx
            parts_k.append(self._tokens(self.kbits, self.kscale, idx))
            parts_v.append(self._tokens(self.vbits, self.vscale, idx))
        if self.tail_k.shape[0]:
            t0 = self.n_tiles * self.tile
            keep = [i for i in range(self.tail_k.shape[0]) if not (exclude_start <= t0 + i < exclude_end)]
            if keep:
                sel = torch.tensor(keep, device=self.device)
                parts_k.append(self.tail_k[sel])
                parts_v.append(self.tail_v[sel])
        if not parts_k:
            return empty
        return torch.cat(parts_k).contiguous(), torch.cat(parts_v).contiguous().half()

    @torch.no_grad()
    def retrieve(self, q_post_rope, n_q=None):
        """Attention of each query head over the segment's top tiles only (fp32 (n_q, d));
        the reference's per-head variant (kvr_retrieval.py:209-232)."""
        n_q = n_q or q_post_rope.shape[0]
        out = torch.zeros(n_q, self.d_head, device=self.device, dtype=torch.float32)
        if self.n_tiles == 0:
            return out
        q, qbar = self._qbar(q_post_rope, n_q)
        k = min(max(1, self.top_k // self.tile), self.n_tiles)
        idx = _hip.topk_tiles(_hip.score_tiles(qbar, self.kbits, self.n_tiles, self.tile), k)
        return _hip.decode_attn(q, None, None, 0, self.kbits, self.vbits, self.kscale, self.vscale, idx,
                                self.tile, self.transform, out_dtype=torch.float32)[0]
