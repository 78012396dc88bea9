"""KVRHook -- window + 1-bit-tile retrieval attention injected into a HuggingFace Llama-style
model through forward hooks (drop-in for the reference's modules/kvr_hook.py:13-331).

API kept: KVRHook(model, window_size=2048, top_k=128, ret_weight=1.0, device=None, **kwargs),
prefill(input_ids), register(), remove(), reset(), _update_stores(li, k_pre, v, k_post),
and the caller-advanced counters `_step` / `_context_len` (callers run
`model(cur, use_cache=False)` then do `hook._step += 1; hook._context_len += 1`, as in
scripts/_niah_64k.py:58-64).  On step 0 the current token is already stored (prefill); on
later steps the hook stores the new token before attending, as the reference does
(kvr_hook.py:250-251).  The attention module's output at the last position is replaced by
o_proj(KVR attention) (kvr_hook.py:309-312); optional "denoise" MLP passes follow the
reference (kvr_hook.py:286-293, default 3 steps; pass num_denoise_steps=0 to disable).

Retargeted to transformers 5.x: RoPE comes from model.model.rotary_emb (applied like HF, in
the model dtype) at the ABSOLUTE position _context_len - 1 of the current token (the
reference used the per-call position_ids, kvr_hook.py:230-236), and prefill calls
model(..., logits_to_keep=1).  Batches of B >= 1 equal-length sequences are supported.
Prefill encodes each layer's K/V into tiles inside the capture hook, so no fp32 copy of all
layers is kept (kvr_hook.py:93-133 kept them all).

Extra kwargs: tile (64 or 128 tokens), transform ('hadamard' or 'dct'), reserve_tokens
(decode tokens the tile stores are sized for at prefill; default 4096 -- beyond it a store
grows, which an already captured graph does not follow).  The reference's warmup_mode /
calibration / MLP adapters are not part of this path.

Per-layer objects: `windows[li]` and `retrievals[li]` are WindowBuffer- / RetrievalIndex-
compatible views of the layer's TileKVCache (kvr_views.py).  Attention is computed in
fp32 and rounded once to the model dtype (bf16 models: the kernel writes bf16 directly).
Failures are loud: every 64th decode step per layer polls the layer's workspace status
and cache error field without blocking, and `check()` does so synchronously; a bounded
wait that gave up or an invalid cache state raises RuntimeError.
"""
from __future__ import annotations

import torch

from . import _hip
from .kvr_cache import TileKVCache
from .kvr_views import CacheRetrievalView, CacheWindowView


def _rotate_half(x):
    d2 = x.shape[-1] // 2
    return torch.cat((-x[..., d2:], x[..., :d2]), dim=-1)


def apply_rope(x, cos, sin):
    """HF convention: x * cos + rotate_half(x) * sin; x [B, heads, L, d], cos/sin [B, L, d]."""
    return x * cos.unsqueeze(1) + _rotate_half(x) * sin.unsqueeze(1)


class KVRHook:
    def __init__(self, model, window_size=2048, top_k=128, ret_weight=1.0, device=None, **kwargs):
        self.model = model
        self.device = device or model.device
        cfg = model.config
        self.n_layers = cfg.num_hidden_layers
        self.n_kv = cfg.num_key_value_heads
        self.n_q = cfg.num_attention_heads
        self.d_head = getattr(cfg, 'head_dim', None) or (cfg.hidden_size // self.n_q)
        if self.d_head != 128:
            raise ValueError("KVRHook's HIP kernels are built for head_dim 128")
        self.g = self.n_q // self.n_kv
        self.window_size = window_size
        self.top_k = top_k
        self._ret_weight = ret_weight
        self.num_denoise_steps = kwargs.get('num_denoise_steps', 3)
        self.chunk_size = kwargs.get('chunk_size', 0)
        self.tile = kwargs.get('tile', 64)
        self.transform = _hip.TRANSFORMS[kwargs.get('transform', 'hadamard')]
        self.reserve_tokens = int(kwargs.get('reserve_tokens', 4096))  # decode tokens the stores are sized for
        for unsupported in ('warmup_mode',):
            if kwargs.get(unsupported):
                raise NotImplementedError(f"{unsupported} is not part of the 1-bit KV path")
        self._context_len = 0
        self._prefill_done = False
        self._hooks = []
        self._step = 0
        self._retrieval_built = False
        self.caches = [None] * self.n_layers

    # The reference exposes per-layer WindowBuffer / RetrievalIndex objects (kvr_hook.py:43-47);
    # here both are views of the layer's TileKVCache (sequence 0; CacheWindowView /
    # CacheRetrievalView take b= for the others).
    @property
    def windows(self):
        return [CacheWindowView(self, li) for li in range(self.n_layers)]

    @property
    def retrievals(self):
        return [CacheRetrievalView(self, li) for li in range(self.n_layers)]

    def _layers(self):
        return self.model.model.layers

    def _dtype(self):
        """Window storage dtype: the model's (bf16, fp16 or fp32)."""
        dt = next(self.model.parameters()).dtype
        return dt if dt in (torch.bfloat16, torch.float16, torch.float32) else torch.float32

    @staticmethod
    def _out_dtype(dt):
        """Attention output dtype: bf16 for bf16 models, else fp32, rounded once to the model
        dtype afterwards (the reference rounds its fp32 attention to the model dtype,
        kvr_hook.py:280)."""
        return torch.bfloat16 if dt == torch.bfloat16 else torch.float32

    def _rope(self, ref, positions):
        """cos, sin [B, L, d] for absolute positions [B, L] (model dtype, as HF)."""
        return self.model.model.rotary_emb(ref, position_ids=positions)

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, input_ids):
        """Full model forward over the prompt; every layer's K/V is captured post-RoPE and split
        into the exact window and the 1-bit tile store as it is produced."""
        B, L = input_ids.shape
        dt = self._dtype()
        extra = max(64, -(-self.reserve_tokens // self.tile) + 1)  # tiles the decode steps will add
        self.caches = [TileKVCache(B, self.n_kv, self.window_size, self.tile, self.transform, self.device, dt,
                                   tile_cap=L // self.tile + extra) for _ in range(self.n_layers)]
        hooks = []

        def make(li):
            def hook(mod, args, kwargs, output):
                hidden = kwargs['hidden_states'] if 'hidden_states' in kwargs else args[0]
                cos, sin = kwargs['position_embeddings']
                k = mod.k_proj(hidden).view(B, L, self.n_kv, self.d_head).transpose(1, 2)
                v = mod.v_proj(hidden).view(B, L, self.n_kv, self.d_head).transpose(1, 2)
                self.caches[li].load_prompt(apply_rope(k, cos, sin), v)
            return hook

        for li, layer in enumerate(self._layers()):
            hooks.append(layer.self_attn.register_forward_hook(make(li), with_kwargs=True))
        try:
            self.model(input_ids, logits_to_keep=1, use_cache=False)
        finally:
            for h in hooks:
                h.remove()
        self._context_len = L
        self._prefill_done = True
        self._retrieval_built = L > self.window_size

    # ------------------------------------------------------------------ stores
    def _update_stores(self, li, k_pre, v_val, k_post):
        """Append the current token (post-RoPE K) to layer li; kvr_hook.py:136-148."""
        B = self.caches[li].B
        self.caches[li].append(k_post.reshape(B, self.n_kv, self.d_head), v_val.reshape(B, self.n_kv, self.d_head))
        self._retrieval_built = self._retrieval_built or self.caches[li].n_tiles > 0

    # ------------------------------------------------------------------ decode hook
    def _make_hook(self, li):
        def hook(mod, args, kwargs, output):
            hidden = kwargs['hidden_states'] if 'hidden_states' in kwargs else args[0]
            B = hidden.shape[0]
            h_last = hidden[:, -1:, :]
            q = mod.q_proj(h_last).view(B, 1, self.n_q, self.d_head).transpose(1, 2)
            k = mod.k_proj(h_last).view(B, 1, self.n_kv, self.d_head).transpose(1, 2)
            v = mod.v_proj(h_last).view(B, 1, self.n_kv, self.d_head)
            pos = torch.full((B, 1), self._context_len - 1, device=hidden.device, dtype=torch.long)
            cos, sin = self._rope(h_last, pos)
            q_rot = apply_rope(q, cos, sin)[:, :, 0]            # [B, Hq, d]
            k_rot = apply_rope(k, cos, sin)[:, :, 0]            # [B, Hkv, d]
            if self._step > 0:
                self._update_stores(li, None, v[:, 0], k_rot)
            cache = self.caches[li]
            top = self.top_k if (self._ret_weight > 0) else 0  # ret_weight <= 0: window only (kvr_hook.py:261)
            attn = cache.attend(q_rot.contiguous(), top, out_dtype=self._out_dtype(hidden.dtype))
            proj = mod.o_proj(attn.reshape(B, 1, self.n_q * self.d_head).to(hidden.dtype))
            if self.num_denoise_steps > 0:
                layer = self._layers()[li]
                h_in = h_last
                h = h_in + proj
                for _ in range(self.num_denoise_steps):
                    h = h + layer.mlp(layer.post_attention_layernorm(h))
                proj = h - h_in
            new_attn = output[0].clone()
            new_attn[:, -1:, :] = proj
            return (new_attn,) + tuple(output[1:])
        return hook

    # ------------------------------------------------------------------ files
    def save_state(self, f):
        """Every layer's cache plus the decode counters (_context_len, _step) as one store
        file (include/kvr_store.h): a prompt's state saved once after prefill can be
        loaded for every request that shares the prompt (prefix caching)."""
        from . import kvr_store
        if not self._prefill_done or any(c is None for c in self.caches):
            raise RuntimeError("nothing to save: run prefill first")
        return kvr_store.save(f, self.caches, user=(self._context_len, self._step, 0, 0))

    def load_state(self, f):
        """Replace every layer's cache and the decode counters with a store file written by
        save_state (same model shape); hooks stay as they are (call register() to decode)."""
        from . import kvr_store
        caches, desc = kvr_store.load(f, self.device, reserve_tiles=-(-self.reserve_tokens // self.tile) + 1,
                                      dtype=self._dtype())
        if (desc.n_layers, desc.Hkv, desc.W, desc.T, desc.transform) != \
           (self.n_layers, self.n_kv, self.window_size, self.tile, self.transform):
            raise ValueError(f"store {desc} does not match this hook (layers={self.n_layers}, n_kv={self.n_kv}, "
                             f"window={self.window_size}, tile={self.tile}, transform={self.transform})")
        self.caches = caches
        self._context_len, self._step = int(desc.user[0]), int(desc.user[1])
        self._prefill_done = True
        self._retrieval_built = desc.n_tiles > 0
        return desc

    def check(self):
        """Synchronising status check of every layer (see the module docstring)."""
        for c in self.caches:
            if c is not None:
                c.check()

    def register(self):
        for li, layer in enumerate(self._layers()):
            self._hooks.append(layer.self_attn.register_forward_hook(self._make_hook(li), with_kwargs=True))

    def remove(self):
        for h in self._hooks:
            h.remove()
        self._hooks = []

    def reset(self):
        self._context_len = 0
        self._prefill_done = False
        self._step = 0
        self._retrieval_built = False
        self.remove()
        self.caches = [None] * self.n_layers

    def __repr__(self):
        ret_state = "ready" if self._retrieval_built else "lazy"
        return (f"KVRHook(layers={self.n_layers}, window={self.window_size}, "
                f"top_k={self.top_k}, ctx={self._context_len}, ret={ret_state})")
