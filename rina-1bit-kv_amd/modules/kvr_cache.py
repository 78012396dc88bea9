"""Per-layer decode state on the GPU: an exact bf16/fp16 window plus the 1-bit tile store.

This is the storage the fused decode kernels read (not part of the reference API; the
reference keeps a fp16 ring per layer in WindowBuffer and an int4 store in RetrievalIndex,
modules/kvr_window.py:9-41, modules/kvr_retrieval.py:150-207).

Layout (head-major so every (sequence, KV head) window is one contiguous run in HBM):
  win_k, win_v : [B, Hkv, W + T, 128]; tokens [0, n) are valid, W <= n < W + T once the
                 store is non-empty (the retrieval region is a multiple of T tokens).
  kbits, vbits : int64 [B * Hkv, tile_cap, 128, T / 64] (uint64 words, bit t = token t)
  kscale,vscale: fp16  [B * Hkv, tile_cap]
  kcount       : uint8 [B * Hkv, tile_cap, 128], each K tile's channel counts (set bits over
                 its T tokens), written with the tile; the decode step scores tiles from it
                 (128 bytes per tile instead of the tile's 128 * T / 8).
When an append fills the window to W + T tokens, its oldest T tokens are encoded into the
next tile slot straight from a strided view of the window, and the remaining W tokens move
down by T (one W-token copy per T decode steps).
"""
from __future__ import annotations

import torch

from . import _hip


class TileKVCache:
    def __init__(self, batch: int, n_kv: int, window: int, tile: int, transform: int,
                 device, dtype=torch.bfloat16, tile_cap: int = 64):
        if window % tile:
            raise ValueError(f"window_size={window} must be a multiple of the tile size {tile}")
        if tile not in (64, 128):
            raise ValueError(f"tile size {tile} unsupported (64 or 128)")
        self.B, self.Hkv, self.W, self.T, self.transform = batch, n_kv, window, tile, transform
        self.device, self.dtype = device, dtype
        cap = window + tile
        self.win_k = torch.zeros((batch, n_kv, cap, 128), dtype=dtype, device=device)
        self.win_v = torch.zeros_like(self.win_k)
        self.n = 0
        self.n_tiles = 0
        self.kbits, self.kscale = _hip.alloc_store(batch * n_kv, tile_cap, tile, device)
        self.vbits, self.vscale = _hip.alloc_store(batch * n_kv, tile_cap, tile, device)
        self.kcount = _hip.alloc_counts(batch * n_kv, tile_cap, device)
        self._ws = None

    # ------------------------------------------------------------------ store growth
    def _ensure_tiles(self, need: int):
        cap = self.kbits.shape[1]
        if need <= cap:
            return
        new_cap = max(need, 2 * cap)
        for name in ("kbits", "vbits"):
            old = getattr(self, name)
            new = torch.zeros((old.shape[0], new_cap) + tuple(old.shape[2:]), dtype=old.dtype, device=old.device)
            new[:, :cap] = old
            setattr(self, name, new)
        for name in ("kscale", "vscale", "kcount"):
            old = getattr(self, name)
            new = torch.zeros((old.shape[0], new_cap) + tuple(old.shape[2:]), dtype=old.dtype, device=old.device)
            new[:, :cap] = old
            setattr(self, name, new)

    def _encode(self, k, v):
        """k, v: [B, Hkv, m*T, 128] (any strides, last dim contiguous) -> tiles appended."""
        m = k.shape[2] // self.T
        if m == 0:
            return
        self._ensure_tiles(self.n_tiles + m)
        _hip.encode_tiles(k, self.T, self.transform, bits=self.kbits, scales=self.kscale, tile_offset=self.n_tiles,
                          counts=self.kcount)
        _hip.encode_tiles(v, self.T, self.transform, bits=self.vbits, scales=self.vscale, tile_offset=self.n_tiles)
        self.n_tiles += m

    # ------------------------------------------------------------------ filling
    def load_prompt(self, k_post, v):
        """Whole prompt: k_post, v [B, Hkv, L, 128] (post-RoPE K).  Tokens beyond the last
        W..W+T-1 go to the store in T-token tiles; the rest fill the window."""
        L = k_post.shape[2]
        n_ret = (L - self.W) // self.T * self.T if L > self.W else 0
        self.n_tiles = 0
        self.n = 0
        if n_ret:
            self._encode(k_post[:, :, :n_ret], v[:, :, :n_ret])
        r = L - n_ret
        self.win_k[:, :, :r] = k_post[:, :, n_ret:].to(self.dtype)
        self.win_v[:, :, :r] = v[:, :, n_ret:].to(self.dtype)
        self.n = r

    def append(self, k_post, v):
        """One token per sequence: k_post, v [B, Hkv, 128]."""
        self.win_k[:, :, self.n] = k_post.to(self.dtype)
        self.win_v[:, :, self.n] = v.to(self.dtype)
        self.n += 1
        if self.n == self.W + self.T:
            self._encode(self.win_k[:, :, :self.T], self.win_v[:, :, :self.T])
            self.win_k[:, :, :self.W] = self.win_k[:, :, self.T:].clone()
            self.win_v[:, :, :self.W] = self.win_v[:, :, self.T:].clone()
            self.n = self.W

    @property
    def n_stored(self) -> int:
        return self.n_tiles * self.T

    # ------------------------------------------------------------------ decode
    def attend(self, q, top_k_tokens: int, out_dtype=torch.bfloat16, out=None, idx_out=None, workspace=None):
        """Decode attention of q [B, Hq, 128] (post-RoPE) over window + top tiles."""
        k = min(max(1, top_k_tokens // self.T), self.n_tiles) if self.n_tiles else 0
        if workspace is None:
            need = _hip.lib().kvr_decode_step_workspace(self.B, q.shape[1], self.Hkv, self.n, self.n_tiles, k,
                                                        self.T)
            if self._ws is None or self._ws.numel() < need:
                # grown geometrically; zeroed before its first call (it holds the launch's counters)
                self._ws = torch.zeros(max(256, 2 * need), dtype=torch.uint8, device=self.device)
            workspace = self._ws
        return _hip.decode_step(q, self.win_k, self.win_v, self.n, self.kbits, self.vbits, self.kscale,
                                self.vscale, self.n_tiles, self.T, self.transform, k, out_dtype=out_dtype,
                                out=out, idx_out=idx_out, workspace=workspace, kcounts=self.kcount)
