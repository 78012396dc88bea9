"""Benchmark of the compressed-KV decode hot path on one MI355X.

Default workload = BASELINE.json configs[2] ("decode32k"): one layer, batch 16, 32768-token
context, GQA 32/8, head_dim 128, bf16 window of the last 1024 tokens, the other 31744 tokens
pre-encoded to 1-bit tiles of 64 (Hadamard-128, sigma-delta), top-32 tiles per KV head.
A step = one call of kvr_decode_step (query prep -> tile scores -> top-k -> fused window +
retrieved-tile attention) over the batch, inputs resident in HBM.  value = decode tokens/s
for that layer (B / step time).

Also reported: encode GB/s at configs[1] (32 layers x 8 KV heads x 16384 tokens, K and V),
the HBM roofline of the decode step, and the CPU oracle timed on a bounded sample.
Synthetic data only (no checkpoints): K = N(0,1) * log-normal(sigma=1) per-channel scales with
RoPE (base 500000) applied, V = N(0,1), q = N(0,1), 16 planted query-aligned keys per sequence.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-encode]
       python bench.py --copy-calibration   (plain copy kernel for rocprof counter scaling)
"""
import argparse
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
                 device="cuda", seed=0, counts=True):
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
    x Hkv heads x N tokens into 1-bit tiles; returns (ms per K+V pair, bytes moved)."""
    K, V = make_kv(n_seq, Hkv, N, 100, "cuda")
    kb, ks = H.alloc_store(n_seq * Hkv, N // T, T, "cuda")
    vb, vs = H.alloc_store(n_seq * Hkv, N // T, T, "cuda")

    def run():
        H.encode_tiles(K, T, tf, bits=kb, scales=ks)
        H.encode_tiles(V, T, tf, bits=vb, scales=vs)

    ms = time_events(run, steps, 2)
    nbytes = 2 * n_seq * Hkv * N * D * 2 + 2 * n_seq * Hkv * N * D // 8 + 2 * n_seq * Hkv * (N // T) * 2
    del K, V, kb, vb
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
    as one async sequence (the generated ids stay on the device)."""
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
    gen = KVRGenerator(model, window_size=2048, top_k=64 * 64)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gen.prefill(ids)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"  e2e prefill of {n_prompt} tokens: {prefill_s:.2f} s")
    gen.step(ids[:, -1:], do_sample=False)  # step 0 (its token is already stored), untimed
    for _ in range(2):
        gen.step(do_sample=False)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n_new):
        gen.step(do_sample=False)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    res = {"e2e_config": f"configs[3]: random-init Llama-3-8B architecture ({n_layers} layers), bf16, batch 1, "
                         f"{n_prompt}-token random prompt, window 2048, top-64 tiles of 64",
           "e2e_prefill_s": round(prefill_s, 3), "e2e_new_tokens": n_new,
           "e2e_decode_ms_per_token": round(ms / n_new, 4),
           "e2e_decode_tokens_per_s": round(n_new / (ms / 1e3), 2),
           "e2e_context_at_end": gen.kvr._context_len}
    del gen, model
    torch.cuda.empty_cache()
    return res


def cpu_baseline(wl, min_seconds=12.0):
    """The numpy oracle on one host core, repeating the whole-batch decode step (query prep,
    scoring of every tile, top-k, float64 attention; all B sequences) until min_seconds of
    CPU work have been timed.  Inputs are copied to host memory first (not timed)."""
    from threadpoolctl import threadpool_limits
    from oracle import kvr_oracle as O
    Hkv = wl.Hkv
    q = wl.q.float().cpu().numpy()
    wk = wl.win_k.float().cpu().numpy()
    wv = wl.win_v.float().cpu().numpy()
    kb = wl.kbits.cpu().numpy().view(np.uint64)
    vb = wl.vbits.cpu().numpy().view(np.uint64)
    ks = wl.kscale.cpu().numpy()
    vs = wl.vscale.cpu().numpy()
    reps = 0
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        while True:
            qbar, _ = O.query_prep(q, Hkv, wl.transform)
            sc = O.score_tiles(qbar.reshape(-1, D), kb)
            idx = O.topk_tiles(sc, wl.k)
            O.decode_attention(q, wk, wv, kb, vb, ks, vs, idx, wl.transform)
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= min_seconds:
                break
    match = bool(np.array_equal(idx, wl.idx.cpu().numpy()))
    return {"value": round(reps * wl.B / dt, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle, 1 thread: {reps} whole-batch decode steps (B={wl.B}; query prep, "
                      f"scores of {wl.n_tiles} tiles x {Hkv} KV heads, top-{wl.k}, float64 attention over "
                      f"{wl.W} window tokens + the selected tiles) in {dt:.1f} s",
            "topk_matches_gpu": match}


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
    ap.add_argument("--no-rotate", action="store_true", help="skip the rotating-layers (HBM-resident) leg")
    ap.add_argument("--no-cfg4", action="store_true", help="skip the configs[4] (DCT, T=128) decode leg")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--e2e", action="store_true", help="also run the configs[3] end-to-end decode leg")
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
    wl = DecodeWorkload()
    log(f"  n_tiles={wl.n_tiles} W={wl.W}; warmup {args.warmup}, timing {args.steps} steps")
    ms = time_events(wl.step, args.steps, args.warmup)
    total, comp = wl.algorithmic_bytes()
    step_gbps = total / ms / 1e6
    log(f"  decode step {ms * 1e3:.1f} us  ({step_gbps:.0f} GB/s algorithmic)")
    # the same step scoring from the K bits instead of the per-tile channel counts
    kc, wl.kcount = wl.kcount, None
    bits_ms = time_events(wl.step, args.steps, args.warmup)
    bits_total, _ = wl.algorithmic_bytes()
    wl.kcount = kc
    log(f"  decode step scoring from the K bits: {bits_ms * 1e3:.1f} us ({bits_total / bits_ms / 1e6:.0f} GB/s algorithmic)")

    # the same step with each step's layer read from HBM (4 layers of stores > the MALL)
    cold_ms = None
    if not args.no_rotate:
        wl.make_layers(4)
        cold_ms = time_events(wl.step_rotating, args.steps, args.warmup)
        del wl.layers
        log(f"  decode step, 4 rotating layers (HBM-resident): {cold_ms * 1e3:.1f} us "
            f"({total / cold_ms / 1e6:.0f} GB/s algorithmic)")

    # DCT-II, T=128, B=4, GQA 28/4, context 131072, window 2048, top-64 tiles
    cfg4 = {}
    if not args.no_cfg4:
        log("building configs[4] workload (B=4, Hq=28, Hkv=4, N=131072, W=2048, T=128, k=64, DCT) ...")
        wl4 = DecodeWorkload(B=4, Hq=28, Hkv=4, N=131072, W=2048, T=128, k=64, transform=H.DCT, seed=4)
        ms4 = time_events(wl4.step, args.steps, args.warmup)
        tot4, comp4 = wl4.algorithmic_bytes()
        cfg4 = {"cfg4_us_per_step": round(ms4 * 1e3, 2), "cfg4_tokens_per_s": round(wl4.B / (ms4 / 1e3), 1),
                "cfg4_algorithmic_bytes": tot4, "cfg4_gbps": round(tot4 / ms4 / 1e6, 1),
                "cfg4_roofline_frac": round(tot4 / ms4 / 1e6 / HBM_PEAK_GBPS, 4)}
        log(f"  configs[4] step {ms4 * 1e3:.1f} us ({tot4 / ms4 / 1e6:.0f} GB/s algorithmic, "
            f"{cfg4['cfg4_roofline_frac'] * 100:.1f} % of 8 TB/s)")
        del wl4
        torch.cuda.empty_cache()

    breakdown = {} if args.no_breakdown else kernel_breakdown(wl, 50)
    if breakdown:
        log("  breakdown (us): " + ", ".join(f"{k}={v * 1e3:.1f}" for k, v in breakdown.items()))
    recall = wl.planted_recall()
    enc = {} if args.no_encode else encode_results(10)
    if enc:
        log(f"  encode configs[1]: {enc['encode_ms']:.3f} ms, {enc['encode_gbps']} GB/s; "
            f"configs[4] layer (DCT, T=128): {enc['cfg4_encode_ms']:.3f} ms, {enc['cfg4_encode_gbps']} GB/s")
    e2e = {}
    if args.e2e:
        log(f"configs[3] end-to-end: {args.e2e_layers} layers, prompt {args.e2e_prompt}, {args.e2e_new} new tokens ...")
        e2e = e2e_benchmark(args.e2e_prompt, args.e2e_new, args.e2e_layers)
        log(f"  e2e decode: {e2e['e2e_decode_tokens_per_s']} tokens/s ({e2e['e2e_decode_ms_per_token']} ms/token)")
    cpu = None if args.no_cpu else cpu_baseline(wl)
    if cpu:
        log(f"  cpu baseline: {cpu['value']} tokens/s ({cpu['sample']})")

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
        "config": {"workload": "configs[2] decode microbench: 1 layer, B=16, ctx 32768, GQA 32/8, d=128, "
                               "bf16 window 1024, 1-bit Hadamard tiles of 64, top-32 tiles",
                   "batch": wl.B, "context": wl.N, "window": wl.W, "tile": wl.T, "top_k_tiles": wl.k,
                   "n_tiles": wl.n_tiles, "transform": "hadamard"},
        "roofline": {"bound": "hbm", "kernel": "kvr::step_kernel (the whole decode step, one launch)",
                     "achieved": round(step_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(step_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": read_traffic("decode_step_decode32k.md"),
                     "algorithmic_bytes": total, "compressed_bytes": comp,
                     "compressed_gbps": round(comp / ms / 1e6, 1)},
        "cpu_baseline": cpu,
        "extra": {"planted_tile_recall": round(recall, 4),
                  "tokens_per_s_32_layers": round(wl.B / (ms / 1e3) / 32, 1),
                  "window_mfma_tflops": round(wl.window_flops() / ms / 1e9, 2),
                  "window_mfma_util_vs_bf16_dense": round(wl.window_flops() / ms / 1e9 / BF16_DENSE_TFLOPS, 5),
                  "scan_bits_us_per_step": round(bits_ms * 1e3, 2),
                  "scan_bits_algorithmic_bytes": bits_total,
                  "scan_bits_gbps": round(bits_total / bits_ms / 1e6, 1),
                  **cfg4, **e2e,
                  "rotating_4_layers_us_per_step": round(cold_ms * 1e3, 2) if cold_ms else None,
                  "rotating_4_layers_gbps": round(total / cold_ms / 1e6, 1) if cold_ms else None, **enc,
                  **{k: round(v, 5) for k, v in breakdown.items()}},
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
