"""WindowBuffer -- ring buffer of the last N tokens' post-RoPE K/V (drop-in for the reference's
modules/kvr_window.py:9-69), attended exactly by the gfx950 window-attention kernel.

Same constructor, attributes (k, v, pos, n, cap), append / batch_append ring semantics and
attention() return convention as the reference.  Additions: `dtype` (fp16 as in the
reference, bf16, or fp32) and `batch` (None keeps the reference's (cap, n_kv, d) layout; an int
gives (batch, cap, n_kv, d) with per-call tensors carrying a leading batch dim).
"""
from __future__ import annotations

import math

import torch

from . import _hip


class WindowBuffer:
    def __init__(self, n_kv, d_head, window_size=2048, device='cuda', dtype=torch.float16, batch=None):
        if d_head != 128:
            raise ValueError("the HIP kernels are built for head_dim 128")
        if dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("window dtype must be float16, bfloat16 or float32")
        self.n_kv = n_kv
        self.d_head = d_head
        self.cap = window_size
        self.batch = batch
        shape = (window_size, n_kv, d_head) if batch is None else (batch, window_size, n_kv, d_head)
        self.k = torch.zeros(shape, device=device, dtype=dtype)
        self.v = torch.zeros(shape, device=device, dtype=dtype)
        self.pos = 0
        self.n = 0

    def _slots(self, x):
        return x if self.batch is None else x.transpose(0, 1)  # token axis first

    @torch.no_grad()
    def append(self, k_post_rope, v):
        """One token: (n_kv, d) (or (batch, n_kv, d)); kvr_window.py:19-25."""
        idx = self.pos % self.cap
        self._slots(self.k)[idx] = k_post_rope.to(self.k.dtype)
        self._slots(self.v)[idx] = v.to(self.v.dtype)
        self.pos += 1
        self.n = min(self.n + 1, self.cap)

    @torch.no_grad()
    def batch_append(self, k_all, v_all):
        """Several tokens (token axis first, or second when batched), evicting the oldest;
        kvr_window.py:27-41."""
        kt, vt = self._slots(k_all), self._slots(v_all)
        n = kt.shape[0]
        ks, vs = self._slots(self.k), self._slots(self.v)
        idx = 0
        remaining = n
        while remaining > 0:
            slot = self.pos % self.cap
            step = min(remaining, self.cap - slot)
            ks[slot:slot + step] = kt[idx:idx + step].to(self.k.dtype)
            vs[slot:slot + step] = vt[idx:idx + step].to(self.v.dtype)
            self.pos += step
            remaining -= step
            idx += step
        self.n = min(self.n + n, self.cap)

    def _kernel_views(self):
        """[B, n_kv, cap, d] strided views of k and v for the kernels."""
        k = self.k.unsqueeze(0) if self.batch is None else self.k
        v = self.v.unsqueeze(0) if self.batch is None else self.v
        return k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)

    @torch.no_grad()
    def attention(self, q_post_rope, n_q=None, scale=None):
        """Exact softmax attention of q (n_q, d) (or (batch, n_q, d)) over the window contents,
        GQA by head groups; returns float32 like kvr_window.py:43-69."""
        n_q = n_q or q_post_rope.shape[-2]
        q = q_post_rope.reshape((1 if self.batch is None else self.batch, n_q, self.d_head))
        if q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            q = q.float()
        if scale is not None and not math.isclose(scale, math.sqrt(self.d_head)):
            q = q.float() * (math.sqrt(self.d_head) / scale)  # the kernel divides by sqrt(d)
        if self.n == 0:
            return torch.zeros(q.shape, device=q.device, dtype=torch.float32).reshape(q_post_rope.shape[:-2] + (n_q, self.d_head))
        wk, wv = self._kernel_views()
        out = _hip.decode_attn(q.contiguous(), wk, wv, self.n, None, None, None, None, None, 64, _hip.NONE,
                               out_dtype=torch.float32)
        return out.reshape(q_post_rope.shape[:-2] + (n_q, self.d_head))
