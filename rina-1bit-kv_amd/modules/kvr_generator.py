"""KVRGenerator -- incremental generation with window + 1-bit-tile attention (drop-in for the
reference's modules/kvr_generator.py:15-173).

API kept: KVRGenerator(model, window_size=2048, top_k=128, device=None), prefill(input_ids),
step(token_id=None, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0) -> next id,
generate(max_new_tokens=100, ...).  The per-layer loop follows kvr_generator.py:78-126
(input_layernorm -> q/k/v -> RoPE -> store -> attention -> o_proj + residual ->
post_attention_layernorm -> MLP + residual), with kvr_cache_append + the fused
kvr_decode_step in place of the store update, retrieve and Triton attention
(kvr_generator.py:84-119).

Changes: the current token sits at absolute position _context_len - 1 (the reference used
_context_len, kvr_generator.py:76); B >= 1 sequences decode together; generated ids stay on
the device (no per-step .item(), kvr_generator.py:156) and `do_sample=False` selects greedy
decoding.  Sampling uses the same HF logits processors as the reference.

HIP graphs (graphs=True, the default): every layer's cache keeps its window length, ring
start and tile count on the device, so once the caches are in steady state one token's
whole forward -- 32 x (norm, projections, RoPE, kvr_cache_append, kvr_decode_step, o_proj,
MLP), final norm, lm_head -- is captured once and replayed for every later token; the
position and the input token are written into the graph's static inputs before each
replay.  A cache whose tile store must grow, or a budget the one-launch step does not take
(more than 64 tiles), runs that step eagerly (and the graph is captured again afterwards).
Decode runs on the generator's own stream, which the caller's stream waits for.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .kvr_hook import KVRHook, apply_rope


class KVRGenerator:
    def __init__(self, model, window_size=2048, top_k=128, device=None, **kwargs):
        self.model = model
        self.device = device or model.device
        cfg = model.config
        self.n_layers = cfg.num_hidden_layers
        self.n_kv = cfg.num_key_value_heads
        self.n_q = cfg.num_attention_heads
        self.d_head = getattr(cfg, 'head_dim', None) or (cfg.hidden_size // self.n_q)
        self.hidden_size = cfg.hidden_size
        self.g = self.n_q // self.n_kv
        self.vocab_size = cfg.vocab_size
        self._step_count = 0
        self._generated = []
        self.use_graphs = bool(kwargs.pop('graphs', True))
        kwargs.setdefault('num_denoise_steps', 0)
        self.kvr = KVRHook(model, window_size=window_size, top_k=top_k, device=device, **kwargs)
        self.window_size = window_size
        self.top_k = top_k
        self.embed = model.model.embed_tokens
        self.final_norm = model.model.norm
        self.lm_head = model.lm_head
        self.layers = model.model.layers
        self._is_first = True
        self.last_logits = None
        self._stream = None
        self._graph = None
        self.graph_replays = 0
        self.graph_captures = 0

    @property
    def _generated_ids(self):
        return [t.tolist() for t in self._generated]

    @torch.no_grad()
    def prefill(self, input_ids):
        """Full forward to build the windows and tile stores (kvr_generator.py:41-47)."""
        self.kvr.prefill(input_ids)
        self._generated = []
        self._step_count = 0
        self._is_first = True
        self._graph = None

    # ------------------------------------------------------------------ one token
    def _forward(self, tok, pos, append: bool):
        """Logits [B, vocab] (fp32) of tokens tok [B, 1] at positions pos [B, 1] (device)."""
        B = tok.shape[0]
        h = self.embed(tok)                                        # [B, 1, hidden]
        cos, sin = self.model.model.rotary_emb(h, position_ids=pos)
        odt = self.kvr._out_dtype(h.dtype)
        for li in range(self.n_layers):
            layer = self.layers[li]
            attn = layer.self_attn
            hn = layer.input_layernorm(h)
            q = attn.q_proj(hn).view(B, 1, self.n_q, self.d_head).transpose(1, 2)
            k = attn.k_proj(hn).view(B, 1, self.n_kv, self.d_head).transpose(1, 2)
            v = attn.v_proj(hn).view(B, self.n_kv, self.d_head)
            q_rot = apply_rope(q, cos, sin)[:, :, 0]
            k_rot = apply_rope(k, cos, sin)[:, :, 0]
            cache = self.kvr.caches[li]
            if append:
                cache.append(k_rot, v)
            o = cache.attend(q_rot.contiguous(), self.top_k, out_dtype=odt)
            h = h + attn.o_proj(o.reshape(B, 1, self.n_q * self.d_head).to(h.dtype))
            h = h + layer.mlp(layer.post_attention_layernorm(h))
        return self.lm_head(self.final_norm(h))[:, -1].float()

    # ------------------------------------------------------------------ graphs
    def _graph_ready(self, B):
        """Whether the next appending step may replay (or capture) the graph."""
        if not self.use_graphs:
            return False
        for c in self.kvr.caches:
            if c.B != B or c.live_k(self.top_k) == 0:
                return False
            if c.n + 1 == c.cap and c.n_tiles >= c.tile_cap:  # the store must grow first
                return False
        return True

    def _capture(self, B):
        caches = self.kvr.caches
        for c in caches:  # allocated (and zeroed) outside the graph: replays must not zero them
            c.workspace(self.n_q, c.live_k(self.top_k))
        mirrors = [(c.n, c.start, c.n_tiles) for c in caches]
        tok = torch.zeros((B, 1), dtype=torch.long, device=self.device)
        pos = torch.zeros((B, 1), dtype=torch.long, device=self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self._stream):
            logits = self._forward(tok, pos, append=True)
        for c, (n, s, t) in zip(caches, mirrors):  # capture launched nothing: undo the mirrors' advance
            c.n, c.start, c.n_tiles = n, s, t
        self._graph = (g, tok, pos, logits, B, [c.version for c in caches])
        self.graph_captures += 1

    def _replay(self, token_id, B):
        g, tok, pos, logits, gB, versions = self._graph if self._graph else (None,) * 6
        if g is None or gB != B or versions != [c.version for c in self.kvr.caches]:
            self._capture(B)
            g, tok, pos, logits, _, _ = self._graph
        tok.copy_(token_id)
        pos.fill_(self.kvr._context_len - 1)
        g.replay()
        for c in self.kvr.caches:
            c._advance_host()
        self.graph_replays += 1
        return logits

    # ------------------------------------------------------------------ API
    @torch.no_grad()
    def step(self, token_id=None, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0,
             do_sample=True):
        """One token per sequence.  The first call takes the last prompt token (already stored)."""
        if token_id is None:
            if not self._generated:
                raise ValueError("First step requires token_id")
            token_id = self._generated[-1]
        if isinstance(token_id, int):
            token_id = torch.tensor([[token_id]], device=self.device)
        token_id = token_id.reshape(-1, 1).to(self.device)
        B = token_id.shape[0]
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=self.device)
        caller = torch.cuda.current_stream()
        self._stream.wait_stream(caller)
        with torch.cuda.stream(self._stream):
            if not self._is_first and self._graph_ready(B):
                logits = self._replay(token_id, B).clone()
            else:
                pos = torch.full((B, 1), self.kvr._context_len - 1, device=self.device, dtype=torch.long)
                logits = self._forward(token_id, pos, append=not self._is_first)
            self.last_logits = logits

            if do_sample:
                from transformers import (LogitsProcessorList, RepetitionPenaltyLogitsProcessor,
                                          TemperatureLogitsWarper, TopKLogitsWarper, TopPLogitsWarper)
                processors = LogitsProcessorList()
                if repetition_penalty != 1.0:
                    processors.append(RepetitionPenaltyLogitsProcessor(repetition_penalty))
                if temperature != 1.0:
                    processors.append(TemperatureLogitsWarper(temperature))
                if top_k > 0:
                    processors.append(TopKLogitsWarper(top_k))
                if top_p < 1.0:
                    processors.append(TopPLogitsWarper(top_p))
                ids = torch.cat(self._generated, dim=1) if self._generated else token_id
                for proc in processors:
                    logits = proc(ids, logits)
                next_id = torch.multinomial(F.softmax(logits, dim=-1), 1)
            else:
                next_id = logits.argmax(dim=-1, keepdim=True)
        caller.wait_stream(self._stream)
        next_id.record_stream(caller)  # allocated on the decode stream, used on the caller's
        self.last_logits.record_stream(caller)
        self._generated.append(next_id)
        self._step_count += 1
        self.kvr._context_len += 1
        self._is_first = False
        return next_id

    @torch.no_grad()
    def generate(self, max_new_tokens=100, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0,
                 do_sample=True):
        """Generate max_new_tokens tokens after step() has been primed (kvr_generator.py:163-173);
        the caches' status is checked (synchronously) at the end."""
        out = []
        for _ in range(max_new_tokens):
            out.append(self.step(temperature=temperature, top_k=top_k, top_p=top_p,
                                 repetition_penalty=repetition_penalty, do_sample=do_sample))
        self.kvr.check()
        return torch.cat(out, dim=1)
