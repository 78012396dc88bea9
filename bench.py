"""Benchmark of the compressed-KV decode hot path on one MI355X.

Default workload = BASELINE.json configs[2] ("decode32k"): one layer, batch 16, 32768-token
context, GQA 32/8, head_dim 128, bf16 window of the last 1024 tokens, the other 31744 tokens
pre-encoded to 1-bit tiles of 64 (Hadamard-128, sigma-delta), top-32 tiles per KV head.
A step = one call of kvr_decode_step (query prep -> tile scores -> top-k -> fused window +
retrieved-tile attention) over the batch, inputs resident in HBM: the steps rotate over
--layers copies of the layer's stores (more than the 256 MB last-level cache holds), so each
step reads its layer from HBM as in a multi-layer decode.  value = decode tokens/s for that
layer (B / step time).  The same step re-reading one layer (MALL-resident) is in extra.

Also reported: encode GB/s at configs[1] (32 layers x 8 KV heads x 16384 tokens, K and V),
configs[4]'s decode step, configs[3] end to end (tokens/s of greedy decode on a random-init
Llama-3-8B-architecture model with a 64k prompt), the HBM roofline of the decode step, and
the CPU oracle on the host cores (1 thread and the box's 16).
Synthetic data only (no checkpoints): K = N(0,1) * log-normal(sigma=1) per-channel scales with
RoPE (base 500000) applied, V = N(0,1), q = N(0,1), 16 planted query-aligned keys per sequence.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-encode] [--no-e2e]
       python bench.py --copy-calibration   (plain copy kernel for rocprof counter scaling)
"""
import argparse
import subprocess
import json
import math
import os
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "rina-1bit-kv_amd"))
sys.path.insert(0, REPO)

from modules import _hip as H  # noqa: E402

METRIC = "decode attn tokens/s @32k ctx b16; compressed-KV HBM GB/s vs roofline"
HBM_PEAK_GBPS = 8000.0
BF16_DENSE_TFLOPS = 2500.0  # MI355X dense bf16 MFMA peak
D = 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- synthetic data

def rope_cos_sin(n_pos, base, device):
    inv = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.int64, device=device).float() / D))
    f = torch.outer(torch.arange(n_pos, device=device, dtype=torch.float32), inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x):
    return torch.cat([-x[..., D // 2:], x[..., :D // 2]], dim=-1)


def make_kv(n_seq, Hkv, N, seed0, device, base=500000.0):
    """K (post-RoPE) and V, bf16 [n_seq, Hkv, N, 128]; K ~ N(0,1) * lognormal per-channel scale."""
    K = torch.empty((n_seq, Hkv, N, D), dtype=torch.bfloat16, device=device)
    V = torch.empty_like(K)
    cos, sin = rope_cos_sin(N, base, device)
    for s in range(n_seq):
        g = torch.Generator(device=device).manual_seed(seed0 + s)
        scale = torch.exp(torch.randn((Hkv, 1, D), generator=g, device=device))
        k = torch.randn((Hkv, N, D), generator=g, device=device) * scale
        K[s] = (k * cos + rotate_half(k) * sin).to(torch.bfloat16)
        V[s] = torch.randn((Hkv, N, D), generator=g, device=device).to(torch.bfloat16)
    return K, V


def plant_keys(K, q, n_plant, n_ret, Hkv, seed, device):
    """Overwrite n_plant tokens per sequence (all KV heads) with (0.8 qhat + 0.2 noise) * rho_h."""
    B, Hq = q.shape[0], q.shape[1]
    g = torch.Generator(device=device).manual_seed(seed)
    qbar = q.float().view(B, Hkv, Hq // Hkv, D).mean(2)
    qhat = qbar / qbar.norm(dim=-1, keepdim=True)
    pos = torch.randint(0, n_ret, (B, n_plant), generator=g, device=device)
    for b in range(B):
        rho = K[b].float().norm(dim=-1).median(dim=-1).values          # [Hkv]
        noise = torch.randn((n_plant, Hkv, D), generator=g, device=device)
        noise = noise / noise.norm(dim=-1, keepdim=True)
        planted = (0.8 * qhat[b][None] + 0.2 * noise) * rho[None, :, None]
        K[b][:, pos[b]] = planted.permute(1, 0, 2).to(torch.bfloat16)
    return pos


class DecodeWorkload:
    def __init__(self, B=16, Hq=32, Hkv=8, N=32768, W=1024, T=64, k=32, transform=H.HADAMARD,
                 device="cuda", seed=0, counts=True, keep_keys=False):
        self.B, self.Hq, self.Hkv, self.N, self.W, self.T, self.k = B, Hq, Hkv, N, W, T, k
        self.transform = transform
        n_ret = (N - W) // T * T
        self.n_tiles = n_ret // T
        self.W = N - n_ret
        g = torch.Generator(device=device).manual_seed(seed + 1000)
        self.q = torch.randn((B, Hq, D), generator=g, device=device).to(torch.bfloat16)
        K, V = make_kv(B, Hkv, N, seed, device)
        self.planted = plant_keys(K, self.q, 16, n_ret, Hkv, seed + 2000, device)
        # the K store's per-tile channel counts are written with its tiles (as TileKVCache does)
        self.kcount = H.alloc_counts(B * Hkv, self.n_tiles, device) if counts else None
        self.kbits, self.kscale = H.encode_tiles(K[:, :, :n_ret], T, transform, counts=self.kcount)
        self.vbits, self.vscale = H.encode_tiles(V[:, :, :n_ret], T, transform)
        self.win_k = K[:, :, n_ret:].contiguous()
        self.win_v = V[:, :, n_ret:].contiguous()
        self.K_ret = K[:, :, :n_ret] if keep_keys else None  # for the exact-tile-mean recall diagnostic
        del K, V
        self.out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=device)
        self.idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=device)
        self.ws = H.decode_step_workspace(B, Hq, Hkv, self.W, self.n_tiles, k, T, device)
        torch.cuda.synchronize()

    def step(self):
        H.decode_step(self.q, self.win_k, self.win_v, self.W, self.kbits, self.vbits, self.kscale,
                      self.vscale, self.n_tiles, self.T, self.transform, self.k, out=self.out,
                      idx_out=self.idx, workspace=self.ws, kcounts=self.kcount)

    def make_layers(self, n_layers):
        """n_layers copies of the layer's stores in separate memory, for a step that rotates
        through them: their total exceeds the 256 MB last-level (MALL) cache, so each step
        reads its layer from HBM, as in a multi-layer decode."""
        self.layers = [(self.win_k, self.win_v, self.kbits, self.vbits, self.kscale, self.vscale, self.kcount)]
        for _ in range(n_layers - 1):
            self.layers.append(tuple(None if t is None else t.clone() for t in self.layers[0]))
        self._li = 0
        torch.cuda.synchronize()

    def step_rotating(self):
        wk, wv, kb, vb, ks, vs, kc = self.layers[self._li]
        self._li = (self._li + 1) % len(self.layers)
        H.decode_step(self.q, wk, wv, self.W, kb, vb, ks, vs, self.n_tiles, self.T, self.transform, self.k,
                      out=self.out, idx_out=self.idx, workspace=self.ws, kcounts=kc)

    def window_flops(self):
        """MFMA work of the window part: QK and PV, 2 flop per multiply-add."""
        return 4 * self.B * self.Hq * self.W * D

    def algorithmic_bytes(self):
        """Per step: the scoring scan (every K tile's 128 channel counts, or all K bits when the
        step scores from the bits) + K,V bits and fp16 scales of the selected tiles + bf16
        window K,V + bf16 q in and out."""
        BH, T, W = self.B * self.Hkv, self.T, self.W
        scan = self.n_tiles * D if self.kcount is not None else self.n_tiles * T * D // 8
        sel = 2 * self.k * T * D // 8 + 2 * 2 * self.k
        win = 2 * W * D * 2
        qo = 2 * self.B * self.Hq * D * 2
        comp = BH * (scan + sel)
        return comp + BH * win + qo, comp

    def planted_recall_exact(self):
        """Recall of the planted keys' tiles when tiles are scored with their exact fp32 mean
        keys (no 1-bit codec): separates the codec's loss from the dilution of a planted key
        in its tile's mean.  A diagnostic in torch on the stored bf16 keys."""
        B, Hkv, T, n = self.B, self.Hkv, self.T, self.n_tiles
        qbar = self.q.float().view(B, Hkv, self.Hq // Hkv, D).mean(2)
        hit = tot = 0
        for b in range(B):
            means = self.K_ret[b].float().view(Hkv, n, T, D).mean(2)              # [Hkv, n, D]
            cos = (means @ qbar[b][:, :, None])[..., 0] / (means.norm(dim=-1) * qbar[b].norm(dim=-1)[:, None] + 1e-8)
            top = cos.topk(self.k, dim=-1).indices.cpu()
            for t in (self.planted[b] // T).tolist():
                for h in range(Hkv):
                    tot += 1
                    hit += int(t in top[h].tolist())
        return hit / max(tot, 1)

    def planted_recall(self):
        idx = self.idx.view(self.B, self.Hkv, self.k).cpu()
        tiles = (self.planted // self.T).cpu()
        hit = tot = 0
        for b in range(self.B):
            for t in tiles[b].tolist():
                for h in range(self.Hkv):
                    tot += 1
                    hit += int(t in idx[b, h].tolist())
        return hit / max(tot, 1)


# ----------------------------------------------------------------------------- timing helpers

def time_events(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def kernel_breakdown(wl, steps):
    """Per-stage event timings of the decode step through the component entry points."""
    qbar = torch.empty((wl.B * wl.Hkv, D), dtype=torch.float32, device="cuda")
    scores = torch.empty((wl.B * wl.Hkv, wl.n_tiles), dtype=torch.float32, device="cuda")
    qb, _ = H.query_prep(wl.q, wl.Hkv, wl.transform, want_q_rot=False)
    t_score = time_events(lambda: H.score_tiles(qb, wl.kbits, wl.n_tiles, wl.T, out=scores), steps, 3)
    idx = torch.empty_like(wl.idx)
    t_topk = time_events(lambda: H.topk_tiles(scores, wl.k, out=idx), steps, 3)
    ws = torch.zeros(1 << 26, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(wl.out)
    t_win = time_events(lambda: H.decode_attn(wl.q, wl.win_k, wl.win_v, wl.W, None, None, None, None,
                                              None, wl.T, wl.transform, torch.bfloat16, ws), steps, 3)
    t_attn = time_events(lambda: H.decode_attn(wl.q, wl.win_k, wl.win_v, wl.W, wl.kbits, wl.vbits,
                                               wl.kscale, wl.vscale, idx, wl.T, wl.transform,
                                               torch.bfloat16, ws), steps, 3)
    t_ret = time_events(lambda: H.decode_attn(wl.q, None, None, 0, wl.kbits, wl.vbits, wl.kscale, wl.vscale,
                                              idx, wl.T, wl.transform, torch.bfloat16, ws), steps, 3)
    del qbar, out
    return {"score_ms": t_score, "topk_ms": t_topk, "window_attn_ms": t_win, "retrieved_attn_ms": t_ret,
            "attn_ms": t_attn}


def encode_benchmark(steps, n_seq=32, Hkv=8, N=16384, T=64, tf=H.HADAMARD):
    """Encode K and V (bf16, K with RoPE and outlier channels) of n_seq sequences (or layers)
    x Hkv heads x N tokens into 1-bit tiles, the K store with its per-tile channel counts (as
    the product's caches keep it); returns (ms per K+V pair, bytes moved)."""
    K, V = make_kv(n_seq, Hkv, N, 100, "cuda")
    kb, ks = H.alloc_store(n_seq * Hkv, N // T, T, "cuda")
    vb, vs = H.alloc_store(n_seq * Hkv, N // T, T, "cuda")
    kc = H.alloc_counts(n_seq * Hkv, N // T, "cuda")

    def run():
        H.encode_tiles(K, T, tf, bits=kb, scales=ks, counts=kc)
        H.encode_tiles(V, T, tf, bits=vb, scales=vs)

    ms = time_events(run, steps, 2)
    nbytes = (2 * n_seq * Hkv * N * D * 2 + 2 * n_seq * Hkv * N * D // 8 + 2 * n_seq * Hkv * (N // T) * 2
              + n_seq * Hkv * (N // T) * D)
    del K, V, kb, vb, kc
    torch.cuda.empty_cache()
    return ms, nbytes


def encode_results(steps):
    """configs[1] (32 layers x 8 KV heads x 16384 tokens, Hadamard, T=64) and one layer of
    configs[4] (B=4 x 4 KV heads x 131072 tokens, DCT-II, T=128)."""
    ms, nbytes = encode_benchmark(steps)
    ms4, nbytes4 = encode_benchmark(steps, n_seq=4, Hkv=4, N=131072, T=128, tf=H.DCT)
    return {"encode_config": "configs[1]: 32 layers x 8 KV heads x 16384 tok, K+V bf16 -> 1-bit T=64",
            "encode_ms": round(ms, 4), "encode_bytes": nbytes, "encode_gbps": round(nbytes / ms / 1e6, 1),
            "cfg4_encode_config": "configs[4], one layer: B=4 x 4 KV heads x 131072 tok, K+V bf16 -> DCT-II 1-bit T=128",
            "cfg4_encode_ms": round(ms4, 4), "cfg4_encode_bytes": nbytes4,
            "cfg4_encode_gbps": round(nbytes4 / ms4 / 1e6, 1)}


def e2e_benchmark(n_prompt=65536, n_new=128, n_layers=32):
    """end-to-end greedy decode with KVRGenerator (window 2048, top-64 tiles of 64,
    Hadamard) on a random-init Llama-3-8B-architecture model in bf16 (32 layers, d_model 4096,
    32/8 heads, FFN 14336, vocab 128256, RoPE base 500000), batch 1, after a prompt of
    uniform random token ids (seed 0).  The prompt goes through the model once (SDPA attention;
    the materialising math backend is switched off so a 64 k prompt never builds N x N scores)
    with every layer's K/V encoded as it is produced; then n_new greedy steps, timed with events
    as one async sequence (the generated ids stay on the device): each token one replay of the
    captured per-token graph, then the same number of steps eagerly for comparison."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from modules import KVRGenerator
    torch.backends.cuda.enable_math_sdp(False)
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=n_layers,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      max_position_embeddings=n_prompt + n_new + 64, rope_theta=500000.0,
                      attn_implementation="sdpa")
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    ids = torch.randint(0, cfg.vocab_size, (1, n_prompt), generator=torch.Generator().manual_seed(0)).cuda()
    gen = KVRGenerator(model, window_size=2048, top_k=64 * 64, reserve_tokens=2 * n_new + 64)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gen.prefill(ids)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"  e2e prefill of {n_prompt} tokens: {prefill_s:.2f} s")
    gen.step(ids[:, -1:], do_sample=False)  # step 0 (its token is already stored), untimed
    for _ in range(2):
        gen.step(do_sample=False)            # the first appending step captures the graph
    torch.cuda.synchronize()

    def timed_steps():
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n_new):
            gen.step(do_sample=False)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    r0 = gen.graph_replays
    ms = timed_steps()
    replays = gen.graph_replays - r0
    gen.use_graphs = False                   # the same steps without the graph, for comparison
    ms_eager = timed_steps()
    gen.kvr.check()
    res = {"e2e_config": f"configs[3]: random-init Llama-3-8B architecture ({n_layers} layers), bf16, batch 1, "
                         f"{n_prompt}-token random prompt, window 2048, top-64 tiles of 64",
           "e2e_prefill_s": round(prefill_s, 3), "e2e_new_tokens": n_new,
           "e2e_decode_ms_per_token": round(ms / n_new, 4),
           "e2e_decode_tokens_per_s": round(n_new / (ms / 1e3), 2),
           "e2e_graph_replays": replays,
           "e2e_decode_tokens_per_s_eager": round(n_new / (ms_eager / 1e3), 2),
           "e2e_context_at_end": gen.kvr._context_len}
    del gen, model
    torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------------------------- CPU baseline

_CPU = {}  # the current CPU workload, inherited by forked pool workers


def _cpu_segments(segs):
    """The numpy oracle's decode step for segments segs (one (sequence, KV head) each): query
    prep, scores of all its tiles, top-k, float64 attention over its window + selected tiles."""
    from oracle import kvr_oracle as O
    d = _CPU
    g, T = d["g"], d["T"]
    for s in segs:
        b, h = divmod(s, d["Hkv"])
        q = d["q"][b:b + 1, h * g:(h + 1) * g]
        qbar, _ = O.query_prep(q, 1, d["tf"])
        sc = O.score_tiles(qbar.reshape(-1, D), d["kb"][s:s + 1])
        idx = O.topk_tiles(sc, d["k"])
        O.decode_attention(q, d["wk"][b:b + 1, h:h + 1], d["wv"][b:b + 1, h:h + 1], d["kb"][s:s + 1],
                           d["vb"][s:s + 1], d["ks"][s:s + 1], d["vs"][s:s + 1], idx, d["tf"])
    return len(segs)


def _cpu_encode(x):
    from oracle import kvr_oracle as O
    O.encode(x, _CPU["T"], _CPU["tf"])
    return 1


def _timed(fn, reps=5):
    """1 warmup + the median of reps runs (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def _cpu_model():
    """The host CPU as lscpu names it (else /proc/cpuinfo), with its AVX-512 capability."""
    name, avx512 = "unknown", False
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and name == "unknown":
                name = line.split(":", 1)[1].strip()
            if line.startswith("flags"):
                avx512 = "avx512f" in line.split()
    except OSError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                name = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return f"{name} ({'AVX-512' if avx512 else 'no AVX-512'})"


def cpu_threads():
    """Host threads for the all-core leg: the box's CPU share (16 per GPU) or fewer."""
    return max(1, min(16, os.cpu_count() or 1))


def cpu_decode(wl, threads):
    """Median seconds of one whole-batch decode step of the numpy oracle over all B*Hkv
    segments, serially (threads = 1) or split over a fork pool of `threads` workers."""
    import multiprocessing as mp
    from threadpoolctl import threadpool_limits
    _CPU.clear()
    _CPU.update(dict(q=wl.q.float().cpu().numpy(), wk=wl.win_k.float().cpu().numpy(),
                     wv=wl.win_v.float().cpu().numpy(), kb=wl.kbits.cpu().numpy().view(np.uint64),
                     vb=wl.vbits.cpu().numpy().view(np.uint64), ks=wl.kscale.cpu().numpy(),
                     vs=wl.vscale.cpu().numpy(), g=wl.Hq // wl.Hkv, Hkv=wl.Hkv, T=wl.T, k=wl.k,
                     tf=wl.transform))
    n_seg = wl.B * wl.Hkv
    with threadpool_limits(limits=1):
        if threads == 1:
            return _timed(lambda: _cpu_segments(range(n_seg)))
        chunks = [list(range(i, n_seg, threads)) for i in range(min(threads, n_seg))]
        with mp.get_context("fork").Pool(len(chunks)) as pool:
            return _timed(lambda: pool.map(_cpu_segments, chunks))


def cpu_encode_layer(threads, n_heads=8, N=16384, T=64, tf=H.HADAMARD):
    """Median seconds to encode one configs[1] layer (K and V of n_heads x N tokens, the
    numpy oracle: Hadamard, scale, sigma-delta, packing), serially or over a pool by head."""
    import multiprocessing as mp
    from threadpoolctl import threadpool_limits
    g = np.random.default_rng(0)
    xs = [(g.standard_normal((1, N, D)) * np.exp(g.standard_normal(D))).astype(np.float32)
          for _ in range(2 * n_heads)]
    _CPU.clear()
    _CPU.update(T=T, tf=tf)
    with threadpool_limits(limits=1):
        if threads == 1:
            return _timed(lambda: [_cpu_encode(x) for x in xs])
        with mp.get_context("fork").Pool(min(threads, len(xs))) as pool:
            return _timed(lambda: pool.map(_cpu_encode, xs))


def cpu_configs0_workload():
    """configs[0] on the host (fp32, built with the oracle codec): B=1, GQA 32/8, 4096 tokens,
    window 512, 56 tiles of 64, top-8."""
    from oracle import kvr_oracle as O

    class W0:
        pass
    w = W0()
    B, Hq, Hkv, N, Wn, T = 1, 32, 8, 4096, 512, 64
    g = np.random.default_rng(0)
    K = (g.standard_normal((B, Hkv, N, D)) * np.exp(g.standard_normal((1, Hkv, 1, D)))).astype(np.float32)
    V = (g.standard_normal((B, Hkv, N, D)) * np.exp(g.standard_normal((1, Hkv, 1, D)))).astype(np.float32)
    n_ret = N - Wn
    kb, ks = O.encode(K[:, :, :n_ret].reshape(B * Hkv, n_ret, D), T, O.HADAMARD)
    vb, vs = O.encode(V[:, :, :n_ret].reshape(B * Hkv, n_ret, D), T, O.HADAMARD)
    w.q = torch.from_numpy(g.standard_normal((B, Hq, D)).astype(np.float32))
    w.win_k, w.win_v = torch.from_numpy(K[:, :, n_ret:]), torch.from_numpy(V[:, :, n_ret:])
    w.kbits, w.vbits = torch.from_numpy(kb.view(np.int64)), torch.from_numpy(vb.view(np.int64))
    w.kscale, w.vscale = torch.from_numpy(ks), torch.from_numpy(vs)
    w.B, w.Hq, w.Hkv, w.T, w.k, w.transform = B, Hq, Hkv, T, 8, O.HADAMARD
    return w


def cpu_baseline(wl, wl4, threads):
    """The CPU restatement (numpy oracle, kind "port") on the host cores: the headline value is
    configs[2]'s whole-batch decode step on `threads` threads (tokens/s); also reported at 1
    thread, and configs[0], configs[4] decode and configs[1] encode (one layer, x 32) at both."""
    model = _cpu_model()
    res = {}
    for th in (1, threads):
        t2 = cpu_decode(wl, th)
        res[f"cfg2_decode_tokens_per_s_{th}t"] = round(wl.B / t2, 3)
        res[f"cfg2_step_s_{th}t"] = round(t2, 4)
        if wl4 is not None:
            t4 = cpu_decode(wl4, th)
            res[f"cfg4_decode_tokens_per_s_{th}t"] = round(wl4.B / t4, 3)
            res[f"cfg4_step_s_{th}t"] = round(t4, 4)
        t0 = cpu_decode(cpu_configs0_workload(), th)
        res[f"cfg0_decode_tokens_per_s_{th}t"] = round(1 / t0, 3)
        heads = 2 if th == 1 else 8  # one thread: a quarter layer, scaled x 4
        te = cpu_encode_layer(th, n_heads=heads) * (8 / heads)
        nbytes = 2 * 8 * 16384 * D * 2 + 2 * 8 * 16384 * D // 8 + 2 * 8 * 256 * 2
        res[f"cfg1_encode_s_32_layers_{th}t"] = round(32 * te, 3)
        res[f"cfg1_encode_gbps_{th}t"] = round(nbytes / te / 1e9, 4)
    return {"value": res[f"cfg2_decode_tokens_per_s_{threads}t"], "unit": "tokens/s", "cores": threads,
            "kind": "port", "cpu": model, "host_cpus": os.cpu_count(),
            "sample": f"numpy oracle (query prep, scores of all {wl.n_tiles} tiles x {wl.Hkv} KV heads, top-{wl.k}, "
                      f"float64 attention over {wl.W} window tokens + the selected tiles) for configs[2]'s whole "
                      f"batch of {wl.B}, over a fork pool of {threads} processes by segment; 1 warmup + median of "
                      "5 runs.  breakdown: the same at 1 thread, configs[0] and configs[4] decode, configs[1] "
                      "encode of one layer (K+V, 8 heads x 16384 tokens; at 1 thread 2 heads x 4) x 32",
            "breakdown": res}


def copy_calibration(nbytes=1 << 30, steps=20):
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    ms = time_events(lambda: dst.copy_(src), steps, 3)
    print(json.dumps({"copy_bytes_each_way": nbytes, "copy_ms": ms, "copy_gbps": 2 * nbytes / ms / 1e6}))


def read_traffic(name):
    """HBM bytes per launch from a committed rocprof --pmc summary (a line 'traffic_bytes: N')."""
    p = os.path.join(REPO, "profiles", name)
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes:"):
            return int(float(line.split(":")[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-encode", action="store_true")
    ap.add_argument("--no-breakdown", action="store_true")
    ap.add_argument("--no-cfg4", action="store_true", help="skip the configs[4] (DCT, T=128) decode leg")
    ap.add_argument("--no-e2e", action="store_true", help="skip the configs[3] end-to-end decode leg")
    ap.add_argument("--layers", type=int, default=4,
                    help="layers of stores the headline step rotates through (their total exceeds the MALL)")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--e2e-prompt", type=int, default=65536)
    ap.add_argument("--e2e-new", type=int, default=128)
    ap.add_argument("--e2e-layers", type=int, default=32)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(collectives are out of scope); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (no CPU fallback for the HIP path)", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    H.lib()
    if args.copy_calibration:
        copy_calibration()
        return

    log("building configs[2] workload (B=16, N=32768, W=1024, T=64, k=32) ...")
    wl = DecodeWorkload(keep_keys=True)
    total, comp = wl.algorithmic_bytes()
    log(f"  n_tiles={wl.n_tiles} W={wl.W}; warmup {args.warmup}, timing {args.steps} steps")
    # headline: each step reads its layer's stores from HBM (the layers rotate; their total
    # exceeds the 256 MB last-level cache), as in a multi-layer decode
    wl.make_layers(args.layers)
    ms = time_events(wl.step_rotating, args.steps, args.warmup)
    step_gbps = total / ms / 1e6
    log(f"  decode step, {args.layers} rotating layers (HBM-resident): {ms * 1e3:.2f} us ({step_gbps:.0f} GB/s algorithmic)")
    del wl.layers
    torch.cuda.empty_cache()
    # the same layer re-read every step (its working set stays in the MALL)
    mall_ms = time_events(wl.step, args.steps, args.warmup)
    log(f"  decode step, one layer re-read (MALL-resident): {mall_ms * 1e3:.2f} us")
    # the same step scoring from the K bits instead of the per-tile channel counts
    kc, wl.kcount = wl.kcount, None
    bits_ms = time_events(wl.step, args.steps, args.warmup)
    bits_total, _ = wl.algorithmic_bytes()
    wl.kcount = kc
    log(f"  decode step scoring from the K bits (MALL-resident): {bits_ms * 1e3:.2f} us")

    # DCT-II, T=128, B=4, GQA 28/4, context 131072, window 2048, top-64 tiles
    cfg4, wl4 = {}, None
    if not args.no_cfg4:
        log("building configs[4] workload (B=4, Hq=28, Hkv=4, N=131072, W=2048, T=128, k=64, DCT) ...")
        wl4 = DecodeWorkload(B=4, Hq=28, Hkv=4, N=131072, W=2048, T=128, k=64, transform=H.DCT, seed=4)
        tot4, comp4 = wl4.algorithmic_bytes()
        wl4.make_layers(6)
        ms4 = time_events(wl4.step_rotating, args.steps, args.warmup)
        del wl4.layers
        torch.cuda.empty_cache()
        ms4_mall = time_events(wl4.step, args.steps, args.warmup)
        cfg4 = {"cfg4_us_per_step": round(ms4 * 1e3, 2), "cfg4_tokens_per_s": round(wl4.B / (ms4 / 1e3), 1),
                "cfg4_algorithmic_bytes": tot4, "cfg4_gbps": round(tot4 / ms4 / 1e6, 1),
                "cfg4_roofline_frac": round(tot4 / ms4 / 1e6 / HBM_PEAK_GBPS, 4),
                "cfg4_mall_resident_us_per_step": round(ms4_mall * 1e3, 2)}
        log(f"  configs[4] step {ms4 * 1e3:.2f} us HBM-resident (6 rotating layers), {ms4_mall * 1e3:.2f} us "
            f"MALL-resident ({tot4 / ms4 / 1e6:.0f} GB/s algorithmic, {cfg4['cfg4_roofline_frac'] * 100:.1f} % of 8 TB/s)")

    breakdown = {} if args.no_breakdown else kernel_breakdown(wl, 50)
    if breakdown:
        log("  breakdown (us): " + ", ".join(f"{k}={v * 1e3:.1f}" for k, v in breakdown.items()))
    recall = wl.planted_recall()
    recall_exact = wl.planted_recall_exact()
    log(f"  planted-tile recall {recall:.3f} (1-bit tiles); {recall_exact:.3f} with exact fp32 tile means")
    enc = {} if args.no_encode else encode_results(10)
    if enc:
        log(f"  encode configs[1]: {enc['encode_ms']:.3f} ms, {enc['encode_gbps']} GB/s; "
            f"configs[4] layer (DCT, T=128): {enc['cfg4_encode_ms']:.3f} ms, {enc['cfg4_encode_gbps']} GB/s")
    cpu = None
    if not args.no_cpu:
        th = cpu_threads()
        log(f"  cpu baseline (numpy oracle, 1 and {th} threads) ...")
        cpu = cpu_baseline(wl, wl4, th)
        cpu["topk_matches_gpu"] = None
        log(f"  cpu baseline: {cpu['value']} tokens/s on {th} threads ({cpu['cpu']}); "
            f"{cpu['breakdown']['cfg2_decode_tokens_per_s_1t']} on 1")
    del wl4
    torch.cuda.empty_cache()
    e2e = {}
    if not args.no_e2e:
        log(f"configs[3] end-to-end: {args.e2e_layers} layers, prompt {args.e2e_prompt}, {args.e2e_new} new tokens ...")
        e2e = e2e_benchmark(args.e2e_prompt, args.e2e_new, args.e2e_layers)
        log(f"  e2e decode: {e2e['e2e_decode_tokens_per_s']} tokens/s ({e2e['e2e_decode_ms_per_token']} ms/token, "
            f"{e2e['e2e_graph_replays']} graph replays)")

    rec = {
        "metric": METRIC,
        "value": round(wl.B / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded K/V/q, RoPE base 500000, 16 planted keys per sequence)",
        "config": {"workload": "configs[2] decode microbench: 1 layer per step, B=16, ctx 32768, GQA 32/8, d=128, "
                               "bf16 window 1024, 1-bit Hadamard tiles of 64, top-32 tiles; the layer's stores "
                               f"read from HBM (steps rotate over {args.layers} layers)",
                   "batch": wl.B, "context": wl.N, "window": wl.W, "tile": wl.T, "top_k_tiles": wl.k,
                   "n_tiles": wl.n_tiles, "transform": "hadamard"},
        "roofline": {"bound": "hbm", "kernel": "kvr::step_kernel<64,bf16,1> (the whole decode step, one launch)",
                     "achieved": round(step_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(step_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": read_traffic("decode_step_decode32k.md"),
                     "algorithmic_bytes": total, "compressed_bytes": comp,
                     "compressed_gbps": round(comp / ms / 1e6, 1)},
        "cpu_baseline": cpu,
        "extra": {"planted_tile_recall": round(recall, 4),
                  "planted_tile_recall_exact_tile_means": round(recall_exact, 4),
                  "tokens_per_s_32_layers": round(wl.B / (ms / 1e3) / 32, 1),
                  "mall_resident_us_per_step": round(mall_ms * 1e3, 2),
                  "mall_resident_tokens_per_s": round(wl.B / (mall_ms / 1e3), 1),
                  "mall_resident_gbps": round(total / mall_ms / 1e6, 1),
                  "window_mfma_tflops": round(wl.window_flops() / ms / 1e9, 2),
                  "window_mfma_util_vs_bf16_dense": round(wl.window_flops() / ms / 1e9 / BF16_DENSE_TFLOPS, 5),
                  "scan_bits_us_per_step": round(bits_ms * 1e3, 2),
                  "scan_bits_algorithmic_bytes": bits_total,
                  "scan_bits_gbps": round(bits_total / bits_ms / 1e6, 1),
                  **cfg4, **e2e, **enc,
                  **{k: round(v, 5) for k, v in breakdown.items()}},
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
