"""Per-layer decode state on the GPU: an exact bf16/fp16/fp32 ring window plus the 1-bit tile
store, with the window length, ring start and tile count kept on the device.

This is the storage the fused decode kernels read (not part of the reference API; the
reference keeps a fp16 ring per layer in WindowBuffer and an int4 store in RetrievalIndex,
modules/kvr_window.py:9-41, modules/kvr_retrieval.py:150-207).

Layout (head-major so every (sequence, KV head) window is one contiguous run in HBM):
  win_k, win_v : [B, Hkv, W + T, 128], a ring: the window's n tokens (oldest first) are in
                 slots (start + i) mod (W + T), i < n; W <= n < W + T once the store is
                 non-empty (the retrieval region is a multiple of T tokens).
  kbits, vbits : int64 [B * Hkv, tile_cap, 128, T / 64] (uint64 words, bit t = token t)
  kscale,vscale: fp16  [B * Hkv, tile_cap]
  kcount       : uint8 [B * Hkv, tile_cap, 128], each K tile's channel counts (set bits over
                 its T tokens), written with the tile; the decode step scores tiles from it
                 (128 bytes per tile instead of the tile's 128 * T / 8).
  state        : int32 [B * Hkv, 4] on the device, per segment {n, start, n_tiles, error}.
Appending a token (kvr_cache_append) writes it into its ring slot and, when the ring fills,
encodes the oldest T tokens into the next tile slot and advances the ring start by T --
all on the device, no copy of the window.  The decode step reads the state from the
device too, so a decode step (append + attend) can be captured once in a HIP graph and
replayed for every token.  The host keeps a mirror of the state (the same rule applied to
the same appends) for sizing and for the Python API.
"""
from __future__ import annotations

import torch

from . import _hip


class TileKVCache:
    def __init__(self, batch: int, n_kv: int, window: int, tile: int, transform: int,
                 device, dtype=torch.bfloat16, tile_cap: int = 64):
        if tile not in (64, 128):
            raise ValueError(f"tile size {tile} unsupported (64 or 128)")
        if window % tile or window < tile:
            raise ValueError(f"window_size={window} must be a positive multiple of the tile size {tile}")
        if dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise ValueError("window dtype must be bfloat16, float16 or float32")
        self.B, self.Hkv, self.W, self.T, self.transform = batch, n_kv, window, tile, transform
        self.device, self.dtype = device, dtype
        self.cap = window + tile
        self.win_k = torch.zeros((batch, n_kv, self.cap, 128), dtype=dtype, device=device)
        self.win_v = torch.zeros_like(self.win_k)
        self.n = 0          # host mirror of the device state
        self.start = 0
        self.n_tiles = 0
        self.state = torch.zeros((batch * n_kv, _hip.STATE_WORDS), dtype=torch.int32, device=device)
        self.kbits, self.kscale = _hip.alloc_store(batch * n_kv, max(1, tile_cap), tile, device)
        self.vbits, self.vscale = _hip.alloc_store(batch * n_kv, max(1, tile_cap), tile, device)
        self.kcount = _hip.alloc_counts(batch * n_kv, max(1, tile_cap), device)
        self._ws = None
        self.version = 0    # bumped whenever a buffer the kernels read is reallocated
        self._calls = 0
        self._pending = None

    # ------------------------------------------------------------------ state
    @property
    def tile_cap(self) -> int:
        return self.kbits.shape[1]

    def _push_state(self):
        """Host mirror -> device state (outside any captured graph)."""
        row = torch.tensor([self.n, self.start, self.n_tiles, 0], dtype=torch.int32)
        self.state.copy_(row.expand(self.B * self.Hkv, -1))

    def _advance_host(self):
        """The state rule of kvr_cache_append for one appended token, on the host mirror."""
        if self.n + 1 == self.cap:
            self.n = self.W
            self.start = (self.start + self.T) % self.cap
            self.n_tiles += 1
        else:
            self.n += 1

    def ensure_tiles(self, need: int):
        """Grow the store to at least `need` tile slots (eager only: the kernels of a
        captured graph keep the old buffers; `version` tells callers to re-capture)."""
        cap = self.kbits.shape[1]
        if need <= cap:
            return
        new_cap = max(need, 2 * cap)
        for name in ("kbits", "vbits", "kscale", "vscale", "kcount"):
            old = getattr(self, name)
            new = torch.zeros((old.shape[0], new_cap) + tuple(old.shape[2:]), dtype=old.dtype, device=old.device)
            new[:, :cap] = old
            setattr(self, name, new)
        self.version += 1

    # ------------------------------------------------------------------ filling
    def load_prompt(self, k_post, v):
        """Whole prompt: k_post, v [B, Hkv, L, 128] (post-RoPE K).  Tokens beyond the last
        W..W+T-1 go to the store in T-token tiles; the rest fill the window."""
        L = k_post.shape[2]
        n_ret = (L - self.W) // self.T * self.T if L > self.W else 0
        m = n_ret // self.T
        self.ensure_tiles(m)
        if m:
            _hip.encode_tiles(k_post[:, :, :n_ret], self.T, self.transform, bits=self.kbits, scales=self.kscale,
                              tile_offset=0, counts=self.kcount)
            _hip.encode_tiles(v[:, :, :n_ret], self.T, self.transform, bits=self.vbits, scales=self.vscale,
                              tile_offset=0)
        r = L - n_ret
        self.win_k[:, :, :r] = k_post[:, :, n_ret:].to(self.dtype)
        self.win_v[:, :, :r] = v[:, :, n_ret:].to(self.dtype)
        self.n, self.start, self.n_tiles = r, 0, m
        self._push_state()

    def append(self, k_post, v):
        """One token per sequence: k_post, v [B, Hkv, 128] -- the ring write and, every T
        tokens, one tile encode, on the device (kvr_cache_append)."""
        if self.n + 1 == self.cap and self.n_tiles >= self.tile_cap:
            self.ensure_tiles(self.n_tiles + 1)
        _hip.cache_append(k_post, v, self.win_k, self.win_v, self.W, self.T, self.transform, self.kbits,
                          self.vbits, self.kscale, self.vscale, self.kcount, self.state)
        self._advance_host()

    @property
    def n_stored(self) -> int:
        return self.n_tiles * self.T

    def window_tokens(self):
        """(K, V) of the window in token order, [B, Hkv, n, 128] (a copy)."""
        idx = (torch.arange(self.n, device=self.win_k.device) + self.start) % self.cap
        return self.win_k[:, :, idx], self.win_v[:, :, idx]

    # ------------------------------------------------------------------ files
    def save(self, f, user=(0, 0, 0, 0)):
        """Write this layer (tiles, K channel counts, window) as a one-layer store file
        (include/kvr_store.h; modules/kvr_store.py)."""
        from . import kvr_store
        return kvr_store.save(f, [self], user=user)

    @classmethod
    def load(cls, f, device, reserve_tiles: int = 64, dtype=None) -> "TileKVCache":
        """The first layer of a store file as a new cache (ring at slot 0)."""
        from . import kvr_store
        caches, _ = kvr_store.load(f, device, reserve_tiles=reserve_tiles, dtype=dtype)
        return caches[0]

    # ------------------------------------------------------------------ decode
    def k_tiles(self, top_k_tokens: int) -> int:
        """Tiles selected per KV head: min(max(1, top_k // T), n_tiles) (kvr_retrieval.py:378);
        none when the budget is 0 (retrieval off, as the reference's ret_weight <= 0)."""
        if top_k_tokens <= 0 or self.n_tiles == 0:
            return 0
        return min(max(1, top_k_tokens // self.T), self.n_tiles)

    def live_k(self, top_k_tokens: int) -> int:
        """k of the live-state launch (capacity-sized; the kernel takes min(k, live n_tiles)),
        or 0 when this budget needs the host-argument path."""
        if top_k_tokens <= 0:
            return 0
        k = max(1, top_k_tokens // self.T)
        if k > 64 or k > self.tile_cap or self.B * self.Hkv > 4096:
            return 0
        return k

    def workspace(self, Hq: int, k: int):
        need = _hip.lib().kvr_decode_step_workspace(self.B, Hq, self.Hkv, self.cap - 1, self.tile_cap, k, self.T)
        if self._ws is None or self._ws.numel() < need:
            # zeroed before its first call (it holds the launch's counters); sized for the
            # capacities, so it serves every later step
            self._ws = torch.zeros(max(256, need), dtype=torch.uint8, device=self.device)
            self.version += 1
        return self._ws

    def attend(self, q, top_k_tokens: int, out_dtype=torch.bfloat16, out=None, idx_out=None, workspace=None,
               live=True):
        """Decode attention of q [B, Hq, 128] (post-RoPE) over window + top tiles.  With
        live=True (and a budget the one-launch step takes) the kernel reads the window
        length, ring start and tile count from the device state, so the call can be
        captured in a graph; otherwise they are passed from the host mirror."""
        Hq = q.shape[1]
        kl = self.live_k(top_k_tokens) if live else 0
        if kl:
            ws = workspace if workspace is not None else self.workspace(Hq, kl)
            out = _hip.decode_step(q, self.win_k, self.win_v, self.cap - 1, self.kbits, self.vbits, self.kscale,
                                   self.vscale, self.tile_cap, self.T, self.transform, kl, out_dtype=out_dtype,
                                   out=out, idx_out=idx_out, workspace=ws, kcounts=self.kcount, win_cap=self.cap,
                                   live_state=self.state)
        else:
            k = self.k_tiles(top_k_tokens)
            ws = workspace if workspace is not None else self.workspace(Hq, k)
            out = _hip.decode_step(q, self.win_k, self.win_v, self.n, self.kbits, self.vbits, self.kscale,
                                   self.vscale, self.n_tiles, self.T, self.transform, k, out_dtype=out_dtype,
                                   out=out, idx_out=idx_out, workspace=ws, kcounts=self.kcount,
                                   win_start=self.start, win_cap=self.cap)
        self._calls += 1
        if self._calls % 64 == 0:
            self.poll_status()
        return out

    # ------------------------------------------------------------------ failure reporting
    def poll_status(self):
        """Non-blocking check of the workspace status word and the state's error field:
        the previous poll's asynchronous copy is read if it has landed (raising if either
        is set), and a new copy is queued.  Skipped while a graph is being captured."""
        if torch.cuda.is_current_stream_capturing():
            return
        if self._pending is not None:
            host, ev = self._pending
            if not ev.query():
                return
            self._pending = None
            self._raise_if(int(host[0]), int(host[1]))
        host = torch.empty(2, dtype=torch.int32, pin_memory=True)
        dev = torch.stack([self._ws[:4].view(torch.int32)[0] if self._ws is not None
                           else torch.zeros((), dtype=torch.int32, device=self.device),
                           self.state[:, 3].max()])
        host.copy_(dev, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._pending = (host, ev)

    def check(self):
        """Blocking check (synchronises): raises RuntimeError if a bounded wait of a decode
        step gave up or an append found an invalid state or a full store."""
        self._pending = None
        ws = int(self._ws[:4].view(torch.int32)[0].item()) if self._ws is not None else 0
        self._raise_if(ws, int(self.state[:, 3].max().item()))

    def _raise_if(self, ws_status: int, state_err: int):
        if ws_status:
            self._ws.zero_()
            raise RuntimeError(f"decode step: a bounded wait gave up (workspace status {ws_status}); outputs since "
                               "the last check are unreliable (affected ones are NaN)")
        if state_err:
            self.state[:, 3] = 0
            why = {1: "an invalid cache state", 2: "a full tile store (evicted tokens were dropped)"}
            raise RuntimeError(f"cache append: {why.get(state_err, f'error {state_err}')}")
