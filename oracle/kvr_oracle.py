"""CPU oracle (numpy) for the 1-bit compressed-KV decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this
module, and only as the checker / the timed CPU restatement.  Nothing on the
product path imports it.

What it restates
----------------
The reference (Misaka477/RINA-1bit-KV) stores evicted tokens as int4 K + a
W-predicted V (modules/kvr_retrieval.py:95-207); the 1-bit tile codec that
replaces it exists only as the frozen specification this build wrote.  The
parts the reference DOES fix are followed here and cited per function:

* HF rotate_half RoPE ................ modules/kvr_retrieval.py:27-37
* GQA-mean query for scoring .......... modules/kvr_retrieval.py:270, 296
* cosine with +1e-8 on each norm ...... modules/kvr_retrieval.py:284-286, 310-312
* tile ("chunk") mean scoring ......... modules/kvr_retrieval.py:291-315
* exclusion -> tile range, k rule ..... modules/kvr_retrieval.py:373-378, 391
* NaN score -> -inf ................... modules/kvr_retrieval.py:287-288, 313-314
* per-KV-head top-k ................... modules/kvr_retrieval.py:379, 392
* one joint softmax, scale 1/sqrt(d) .. modules/kvr_hook.py:274-282,
                                        modules/kvr_triton.py:56-79

Codec (frozen here; the kernels implement exactly this)
-------------------------------------------------------
d = 128 channels (head_dim), tiles of T in {64, 128} consecutive tokens.
1. Rotation along head_dim, per token: orthonormal Hadamard-128 (Sylvester,
   natural order) as an fp32 FWHT with stages h = 1, 2, 4, ..., 64 in that
   order, then one fp32 multiply by C_HAD = fp32(2**-3.5) = 0x3db504f3; or the
   orthonormal DCT-II-128 (tolerance only).
2. Tile scale s = fp16_rne(sat(A * 2**-log2(T*128))), A = sum |y| with a fixed
   order: per channel a sequential fp32 sum over t ascending, then a
   stride-halving tree over channels (j += j+64, j+32, ..., j+1); sat(m) = m if
   m < 65504 else 65504.  One scale per (segment, tile), separately for K, V.
3. Sigma-delta along tokens, per channel, e0 = +0 at each tile start:
   u = fl(y + e); b = (u >= 0); q = b ? s32 : -s32 (s32 = float(s)); e = fl(u - q).
4. Packing: word[tile][channel][w] (uint64, w = 0..T/64-1), bit (t mod 64) of
   word w = t // 64 holds b for token t (LSB = first token).
5. Tile score: c_j = 2*popc(word_j) - T; q = rotate(mean_g(q_post)) in fp32;
   score = dot / (fl(sqrt(qq)) + 1e-8f) * (fl(sqrt(cc)) + 1e-8f) with the exact
   fp32 order emulated in score_tiles(); NaN -> -inf; excluded tiles -> -inf.
6. Top-k per segment: score descending, ties by tile index ascending.
7. Attention: one softmax over window tokens (bf16/fp16 K,V) and the tokens of
   the selected tiles, whose keys/values are s*(2b-1) in the rotated domain;
   q' = R q; o = sum_w p v + R^T sum_r p v'; logits scaled by 1/sqrt(d).

Pinning (what checks each function independently of its own formula)
--------------------------------------------------------------------
fwht/hadamard_rotate : H H^T = I (float64), dense Sylvester matrix product,
                       brute force d in {2,4,8}, scipy.linalg.hadamard.
dct_matrix/rotate    : scipy.fft.dct(norm='ortho'), C C^T = I.
tile_scale           : hand-computed KATs, order-independence on exact inputs,
                       float64 mean within fp16 rounding.
sigma_delta_pack     : tile-sum identity sum(q) = sum(y) + e0 - e_T (exact in
                       reals), |e| <= s when |y| <= s, constant-input bit
                       density, hand-written KAT words, brute-force scalar loop.
unpack/pack          : round trip, hand-written words.
score_tiles          : float64 brute force on unpacked +-1 bits (no popcount),
                       the reference's dequantise->chunk-mean->cosine definition.
topk_tiles           : full sort by (score desc, index asc) on brute force.
decode_attention     : torch scaled_dot_product_attention (library routine) on
                       the dequantised, inverse-rotated tokens.
gqa_mean             : torch view(...).mean(1) as at kvr_retrieval.py:270.
rope                 : transformers' LlamaRotaryEmbedding + apply_rotary_pos_emb.
exclusion_to_tiles   : hand-computed cases of kvr_retrieval.py:373-377.
"""
from __future__ import annotations

import numpy as np

D = 128
C_HAD = np.uint32(0x3DB504F3).view(np.float32)  # fp32(2**-3.5)
EPS = np.float32(1e-8)
FP16_MAX = np.float32(65504.0)
HADAMARD = 0
DCT = 1
NONE = 2


# ----------------------------------------------------------------------------- dtype helpers

def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def bf16_to_bits(x) -> np.ndarray:
    """float32 values already representable in bf16 -> uint16 bit patterns."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_bf16(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- RoPE (reference convention)

def rope_tables(n_pos: int, d: int = D, base: float = 500000.0, start: int = 0):
    """cos/sin tables (n_pos, d) float32 in HF Llama layout (freqs duplicated over halves).

    Follows the tables the reference takes from ``rotary_emb`` (kvr_hook.py:49-55):
    inv_freq = base ** -(2i/d), emb = cat(freqs, freqs).  Computed in float32 as HF does.
    """
    inv_freq = (1.0 / (np.float32(base) ** (np.arange(0, d, 2, dtype=np.int64).astype(np.float32) / np.float32(d)))).astype(np.float32)
    pos = np.arange(start, start + n_pos, dtype=np.float32)
    freqs = np.outer(pos, inv_freq).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def rotate_half(x):
    """kvr_retrieval.py:27-29: cat(-x[..., d/2:], x[..., :d/2])."""
    d2 = x.shape[-1] // 2
    return np.concatenate([-x[..., d2:], x[..., :d2]], axis=-1)


def apply_rotary(x, cos, sin):
    """kvr_retrieval.py:32-33: x*cos + rotate_half(x)*sin (cos/sin broadcast over heads)."""
    return x * cos + rotate_half(x) * sin


def reverse_rotary(x, cos, sin):
    """kvr_retrieval.py:36-37."""
    return x * cos - rotate_half(x) * sin


# ----------------------------------------------------------------------------- transforms

def fwht(x, dtype=np.float32):
    """Unnormalised Walsh-Hadamard transform of the last axis (length 128), Sylvester order.

    Stages h = 1, 2, 4, ..., 64 in that order; stage h maps (x[j], x[j+h]) for (j & h) == 0
    to (x[j] + x[j+h], x[j] - x[j+h]).  In float32 each add/sub rounds once (RNE), which is
    exactly what the HIP encoder does, so the result is bit-identical to the kernel.
    """
    x = np.array(x, dtype=dtype, copy=True)
    n = x.shape[-1]
    lead = x.shape[:-1]
    h = 1
    while h < n:
        x = x.reshape(lead + (n // (2 * h), 2, h))
        a = x[..., 0, :]
        b = x[..., 1, :]
        x = np.stack([a + b, a - b], axis=-2).reshape(lead + (n,))
        h *= 2
    return x


def hadamard_rotate(x):
    """Orthonormal Hadamard-128 in the kernel's fp32 order: fl(FWHT(x) * C_HAD)."""
    return (fwht(np.asarray(x, dtype=np.float32)) * C_HAD).astype(np.float32)


def dct_matrix(n: int = D) -> np.ndarray:
    """Orthonormal DCT-II matrix C[k, m] = a_k cos(pi (2m+1) k / 2n), float64."""
    k = np.arange(n)[:, None].astype(np.float64)
    m = np.arange(n)[None, :].astype(np.float64)
    c = np.cos(np.pi * (2 * m + 1) * k / (2 * n))
    c *= np.sqrt(2.0 / n)
    c[0, :] = np.sqrt(1.0 / n)
    return c


def rotate(x, transform: int):
    """Forward rotation of the last axis; fp32 result.  Hadamard is bit-exact to the
    kernel; DCT is the float64 product rounded once (the kernel is within tolerance)."""
    if transform == HADAMARD:
        return hadamard_rotate(x)
    if transform == DCT:
        return (np.asarray(x, dtype=np.float64) @ dct_matrix().T).astype(np.float32)
    if transform == NONE:
        return np.asarray(x, dtype=np.float32)
    raise ValueError(transform)


def rotate64(x, transform: int):
    """Forward rotation in float64 (reference arithmetic for attention)."""
    x = np.asarray(x, dtype=np.float64)
    if transform == HADAMARD:
        return fwht(x, np.float64) / np.sqrt(128.0)
    if transform == DCT:
        return x @ dct_matrix().T
    return x


def inverse_rotate64(y, transform: int):
    """Inverse rotation in float64: H is symmetric orthonormal; DCT-II inverse is C^T."""
    y = np.asarray(y, dtype=np.float64)
    if transform == HADAMARD:
        return fwht(y, np.float64) / np.sqrt(128.0)
    if transform == DCT:
        return y @ dct_matrix()
    return y


# ----------------------------------------------------------------------------- codec

def tile_scale(y) -> np.ndarray:
    """fp16 scale per tile.  y: [..., T, 128] float32 (rotated) -> [...] float16."""
    y = np.asarray(y, dtype=np.float32)
    T = y.shape[-2]
    a = np.abs(y)
    S = np.zeros(a.shape[:-2] + (D,), np.float32)
    for t in range(T):
        S = S + a[..., t, :]
    h = D // 2
    while h >= 1:
        S = S[..., :h] + S[..., h:2 * h]
        h //= 2
    A = S[..., 0]
    m = (A * np.float32(1.0 / (T * D))).astype(np.float32)
    m = np.where(m < FP16_MAX, m, FP16_MAX).astype(np.float32)
    return m.astype(np.float16)


def sigma_delta_pack(y, s16) -> np.ndarray:
    """Sigma-delta 1-bit code of one tile per leading index.

    y: [..., T, 128] float32 rotated values, s16: [...] float16 scales.
    Returns uint64 words [..., 128, T//64].
    """
    y = np.asarray(y, dtype=np.float32)
    T = y.shape[-2]
    W = T // 64
    s = np.asarray(s16, dtype=np.float16).astype(np.float32)[..., None]
    e = np.zeros(y.shape[:-2] + (D,), np.float32)
    words = np.zeros(y.shape[:-2] + (D, W), np.uint64)
    for t in range(T):
        u = y[..., t, :] + e
        b = u >= 0
        q = np.where(b, s, -s)
        e = u - q
        words[..., t // 64] |= b.astype(np.uint64) << np.uint64(t % 64)
    return words


def encode_tiles(y, T: int):
    """Encode rotated fp32 tokens.  y: [S, n_tok, 128] -> (bits [S, n_tiles, 128, T//64] u64,
    scales [S, n_tiles] f16).  n_tok must be a multiple of T."""
    y = np.asarray(y, dtype=np.float32)
    S, n_tok, d = y.shape
    assert d == D and n_tok % T == 0
    yt = y.reshape(S, n_tok // T, T, D)
    s = tile_scale(yt)
    return sigma_delta_pack(yt, s), s


def encode(x, T: int, transform: int):
    """Rotate then encode.  x: [S, n_tok, 128] (values of the input dtype)."""
    return encode_tiles(rotate(x, transform), T)


def unpack_bits(bits) -> np.ndarray:
    """uint64 words [..., 128, W] -> bits [..., 64*W, 128] uint8 (token-major)."""
    bits = np.asarray(bits, dtype=np.uint64)
    W = bits.shape[-1]
    t = np.arange(64, dtype=np.uint64)
    b = (bits[..., None] >> t) & np.uint64(1)           # [..., 128, W, 64]
    b = b.reshape(bits.shape[:-2] + (D, W * 64))         # token index = 64 w + t
    return np.swapaxes(b, -1, -2).astype(np.uint8)


def pack_bits(b) -> np.ndarray:
    """Inverse of unpack_bits: [..., T, 128] {0,1} -> [..., 128, T//64] uint64."""
    b = np.asarray(b, dtype=np.uint64)
    T = b.shape[-2]
    W = T // 64
    bt = np.swapaxes(b, -1, -2).reshape(b.shape[:-2] + (D, W, 64))
    sh = np.arange(64, dtype=np.uint64)
    return np.bitwise_or.reduce(bt << sh, axis=-1)


def dequantize(bits, scales) -> np.ndarray:
    """Rotated-domain reconstruction s*(2b-1): [..., T, 128] float64."""
    b = unpack_bits(bits).astype(np.float64)
    s = np.asarray(scales, dtype=np.float16).astype(np.float64)
    return s[..., None, None] * (2.0 * b - 1.0)


# ----------------------------------------------------------------------------- query side

def gqa_mean(q, n_kv: int):
    """q: [..., Hq, 128] float32 -> [..., Hkv, 128]: sequential fp32 sum over the g heads of
    each group, then one correctly rounded division by g (kvr_retrieval.py:270 mean(dim=1))."""
    q = np.asarray(q, dtype=np.float32)
    Hq = q.shape[-2]
    g = Hq // n_kv
    qg = q.reshape(q.shape[:-2] + (n_kv, g, D))
    acc = qg[..., 0, :].copy()
    for i in range(1, g):
        acc = acc + qg[..., i, :]
    return (acc / np.float32(g)).astype(np.float32)


def query_prep(q, n_kv: int, transform: int):
    """-> (qbar_rot [..., Hkv, 128] f32, q_rot [..., Hq, 128] f32)."""
    return rotate(gqa_mean(q, n_kv), transform), rotate(q, transform)


# ----------------------------------------------------------------------------- scoring

def exclusion_to_tiles(exclude_start: int, exclude_end: int, T: int, n_tiles: int):
    """Token range [start, end) -> tile range [lo, hi) as kvr_retrieval.py:373-377."""
    lo = exclude_start // T
    hi = min((exclude_end + T - 1) // T, n_tiles)
    if lo >= hi:
        lo = hi = 0
    return lo, hi


def tile_colsums(bits) -> np.ndarray:
    """c_j = 2*popc(word_j) - T per tile: [..., 128, W] -> [..., 128] int32."""
    bits = np.asarray(bits, dtype=np.uint64)
    W = bits.shape[-1]
    pc = np.bitwise_count(bits).astype(np.int32).sum(axis=-1)
    return 2 * pc - 64 * W


def _tree16(p):
    """Stride-halving tree over the last axis of length 16 (h = 8, 4, 2, 1)."""
    h = 8
    while h >= 1:
        p = p[..., :h] + p[..., h:2 * h]
        h //= 2
    return p[..., 0]


def _lane_dot(a, b):
    """Kernel order for a 128-term fp32 dot: 16 lanes x 8 channels; per lane a sequential
    sum of fl(a*b) over its 8 consecutive channels, then the 16-lane tree."""
    prod = (a * b).astype(np.float32)
    prod = prod.reshape(prod.shape[:-1] + (16, 8))
    p = prod[..., 0]
    for k in range(1, 8):
        p = p + prod[..., k]
    return _tree16(p)


def score_tiles(qbar_rot, bits, excl=None):
    """Exact fp32 emulation of the HIP tile scorer.

    qbar_rot: [S, 128] float32, bits: [S, n_tiles, 128, W] uint64,
    excl: optional (lo [S], hi [S]) tile ranges set to -inf.
    Returns scores [S, n_tiles] float32.
    """
    q = np.asarray(qbar_rot, dtype=np.float32)
    c = tile_colsums(bits)                                    # [S, n, 128]
    cf = c.astype(np.float32)
    dot = _lane_dot(q[:, None, :], cf)                          # [S, n]
    qq = _lane_dot(q, q)                                        # [S]
    cc = (c.astype(np.int64) ** 2).sum(-1).astype(np.float32)   # exact
    qn = (np.sqrt(qq) + EPS).astype(np.float32)
    cn = (np.sqrt(cc) + EPS).astype(np.float32)
    den = (qn[:, None] * cn).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        sc = (dot / den).astype(np.float32)
    sc = np.where(np.isnan(sc), np.float32(-np.inf), sc)
    if excl is not None:
        lo, hi = excl
        n = sc.shape[1]
        t = np.arange(n)[None, :]
        m = (t >= np.asarray(lo)[:, None]) & (t < np.asarray(hi)[:, None])
        sc = np.where(m, np.float32(-np.inf), sc)
    return sc


def score_tiles_bruteforce(qbar_rot, bits):
    """float64 cosine of qbar' with the column sums of the unpacked +-1 tile (no popcount)."""
    pm = 2.0 * unpack_bits(bits).astype(np.float64) - 1.0       # [S, n, T, 128]
    c = pm.sum(axis=-2)
    q = np.asarray(qbar_rot, dtype=np.float64)
    dot = np.einsum("sd,snd->sn", q, c)
    return dot / ((np.linalg.norm(q, axis=-1)[:, None] + 1e-8) * (np.linalg.norm(c, axis=-1) + 1e-8))


def score_tiles_reference_def(qbar_rot, bits, scales):
    """The reference's chunk definition (kvr_retrieval.py:305-312) on dequantised tiles:
    normalise q and the chunk-mean key with +1e-8 each, then dot (float64)."""
    kmean = dequantize(bits, scales).mean(axis=-2)              # [S, n, 128]
    q = np.asarray(qbar_rot, dtype=np.float64)
    qn = q / (np.linalg.norm(q, axis=-1, keepdims=True) + 1e-8)
    kn = kmean / (np.linalg.norm(kmean, axis=-1, keepdims=True) + 1e-8)
    return np.einsum("sd,snd->sn", qn, kn)


def topk_tiles(scores, k: int):
    """Per-row top-k: score descending, tile index ascending on ties.  -> int32 [S, k]."""
    scores = np.asarray(scores, dtype=np.float32)
    scores = np.where(np.isnan(scores), np.float32(-np.inf), scores)
    S, n = scores.shape
    out = np.empty((S, k), np.int32)
    idx = np.arange(n)
    for s in range(S):
        order = np.lexsort((idx, -scores[s].astype(np.float64)))
        out[s] = order[:k]
    return out


def k_tiles(top_k: int, T: int, n_tiles: int) -> int:
    """kvr_retrieval.py:378: min(max(1, top_k // cs), n_chunks)."""
    return min(max(1, top_k // T), n_tiles)


# ----------------------------------------------------------------------------- attention

def decode_attention(q, win_k, win_v, kbits, vbits, kscale, vscale, idx, transform: int,
                     win_len=None):
    """float64 reference of the fused decode attention.

    q: [B, Hq, 128] (input values), win_k/win_v: [B, Hkv, W, 128] stored window values,
    kbits/vbits: [B*Hkv, n_tiles, 128, Wd] uint64, kscale/vscale: [B*Hkv, n_tiles] f16,
    idx: [B*Hkv, k] int32 (k may be 0), win_len: tokens of the window used (default all).
    Returns out [B, Hq, 128] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    B, Hq, d = q.shape
    Hkv = win_k.shape[1]
    g = Hq // Hkv
    nw = win_k.shape[2] if win_len is None else int(win_len)
    kw = np.asarray(win_k, dtype=np.float64)[:, :, :nw]
    vw = np.asarray(win_v, dtype=np.float64)[:, :, :nw]
    out = np.zeros((B, Hq, d))
    scale = 1.0 / np.sqrt(d)
    for b in range(B):
        for h in range(Hkv):
            s = b * Hkv + h
            sel = np.asarray(idx[s]) if idx is not None else np.zeros(0, np.int32)
            if sel.size:
                kr = dequantize(kbits[s][sel], kscale[s][sel]).reshape(-1, d)
                vr = dequantize(vbits[s][sel], vscale[s][sel]).reshape(-1, d)
            else:
                kr = np.zeros((0, d))
                vr = np.zeros((0, d))
            for i in range(g):
                qh = q[b, h * g + i]
                qr = rotate64(qh, transform)
                lw = kw[b, h] @ qh * scale
                lr = kr @ qr * scale
                allv = np.concatenate([lw, lr])
                if allv.size == 0:
                    continue
                m = allv.max()
                pw = np.exp(lw - m)
                pr = np.exp(lr - m)
                L = pw.sum() + pr.sum()
                o = pw @ vw[b, h] + inverse_rotate64(pr @ vr, transform)
                out[b, h * g + i] = o / L
    return out


def dequantize_original(bits, scales, transform: int):
    """Tokens of tiles reconstructed in the original (unrotated) domain: [..., T, 128] f64."""
    return inverse_rotate64(dequantize(bits, scales), transform)
