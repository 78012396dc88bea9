"""GPU parity at the benchmark configurations' full sizes, through the C ABI.

configs[2] (B=16, GQA 32/8, 32768-token context, bf16 window 1024, Hadamard tiles of 64,
top-32) and configs[4] (B=4, GQA 28/4, 131072-token context, window 2048, DCT tiles of 128,
top-64): the one-launch decode step against the CPU oracle on the same stored inputs --
every segment's selected tiles, and every head's output within the attention tolerance --
scoring from the K store's per-tile channel counts (the product path) and from the bits.
Encoders at full size (configs[1]: 32 layers x 8 KV heads x 16384 tokens; one configs[4]
layer: 4 x 4 x 131072 tokens): sampled segments bit-exact against the oracle codec
(Hadamard from the input, DCT given the kernel's own rotation, which is held to 1e-6 of
the float64 rotation).  Inputs are generated on the GPU (seeded torch generators), so the
tests run in seconds.
"""
import numpy as np
import pytest
import torch

from oracle import kvr_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def H():
    from modules import _hip
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    _hip.lib()
    return _hip


def gen_kv(shape, seed, outliers=True):
    """bf16 N(0,1) values on the GPU, times log-normal(sigma=1) per-channel scales."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=DEV)
    if outliers:
        x *= torch.exp(torch.randn(shape[-1], generator=g, device=DEV))
    return x.to(torch.bfloat16)


def u64(t):
    return t.cpu().numpy().view(np.uint64)


def check_out(out, ref, what):
    o = out.float().cpu().numpy()
    if out.dtype == torch.float32:
        err = np.abs(o - ref).max()
        assert err <= 1e-5, f"{what}: fp32 max-abs {err}"
    else:
        excess = (np.abs(o - ref) - (2e-3 + np.abs(ref) * 2.0 ** -8)).max()
        assert excess <= 0, f"{what}: bf16 error exceeds 2e-3 + 2^-8|ref| by {excess}"


def topk_agree(ig, iref, sref, k, exact):
    if exact:
        assert np.array_equal(ig, iref)
        return
    for s in range(ig.shape[0]):  # rotation held to a tolerance: equal up to near-ties at the k-th score
        if not np.array_equal(np.sort(ig[s]), np.sort(iref[s])):
            kth = np.sort(sref[s])[::-1][k - 1]
            diff = set(ig[s].tolist()) ^ set(iref[s].tolist())
            assert all(abs(sref[s][t] - kth) <= 1e-6 * np.abs(sref[s]).max() for t in diff), s


@pytest.mark.parametrize(
    "cfg,B,Hq,Hkv,N,W,T,k,tf",
    [("configs[2]", 16, 32, 8, 32768, 1024, 64, 32, O.HADAMARD),
     ("configs[4]", 4, 28, 4, 131072, 2048, 128, 64, O.DCT)])
@pytest.mark.parametrize("odt,use_counts", [(torch.bfloat16, True), (torch.float32, True), (torch.float32, False)])
def test_decode_step_full_size(H, cfg, B, Hq, Hkv, N, W, T, k, tf, odt, use_counts):
    say(f"[fullsize/decode_step] {cfg} B={B} Hq={Hq} Hkv={Hkv} N={N} W={W} T={T} k={k} out={odt} "
        f"counts={use_counts}")
    n_tiles = (N - W) // T
    K = gen_kv((B, Hkv, n_tiles * T, 128), 10)
    V = gen_kv((B, Hkv, n_tiles * T, 128), 11, outliers=False)
    counts = H.alloc_counts(B * Hkv, n_tiles, DEV) if use_counts else None
    kb, ks = H.encode_tiles(K, T, tf, counts=counts)
    vb, vs = H.encode_tiles(V, T, tf)
    del K, V
    wk = gen_kv((B, Hkv, W, 128), 12)
    wv = gen_kv((B, Hkv, W, 128), 13, outliers=False)
    q = gen_kv((B, Hq, 128), 14, outliers=False)
    idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
    out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=odt, idx_out=idx,
                        kcounts=counts)
    torch.cuda.synchronize()
    kbn, vbn, ksn, vsn = u64(kb), u64(vb), ks.cpu().numpy(), vs.cpu().numpy()
    qn = q.float().cpu().numpy()
    qbar, _ = O.query_prep(qn, Hkv, tf)
    sref = O.score_tiles(qbar.reshape(-1, 128), kbn)
    iref = O.topk_tiles(sref, k)
    ig = idx.cpu().numpy()
    topk_agree(ig, iref, sref, k, exact=(tf == O.HADAMARD))
    ref = O.decode_attention(qn, wk.float().cpu().numpy(), wv.float().cpu().numpy(), kbn, vbn, ksn, vsn, ig, tf)
    check_out(out, ref, cfg)


def test_encode_full_size_configs1(H):
    """32 layers x 8 KV heads x 16384 tokens (K-like, with outlier channels), Hadamard, T=64:
    four sampled (layer, head) segments bit-exact against the oracle codec."""
    say("[fullsize/encode] configs[1] 32 x 8 x 16384, Hadamard T=64")
    T = 64
    x = gen_kv((32, 8, 16384, 128), 20)
    bits, scales = H.encode_tiles(x, T, O.HADAMARD)
    torch.cuda.synchronize()
    segs = [0, 77, 150, 255]  # segment = layer * 8 + head
    xs = x.view(256, 16384, 128)[segs].float().cpu().numpy()
    rb, rs = O.encode(xs, T, O.HADAMARD)
    gb = bits.view(256, -1)[segs].cpu().numpy().view(np.uint64).reshape(rb.shape)
    gs = scales[segs].cpu().numpy().view(np.uint16)
    assert np.array_equal(gb, rb)
    assert np.array_equal(gs, rs.view(np.uint16))


def test_encode_full_size_configs4_dct(H):
    """One configs[4] layer (B=4 x 4 KV heads x 131072 tokens), DCT-II, T=128: the rotation of
    two sampled segments within 1e-6 of the float64 rotation (relative to the token norm), and
    their bits and scales exact given the rotation the kernel wrote."""
    say("[fullsize/encode] configs[4] layer 4 x 4 x 131072, DCT T=128")
    T = 128
    x = gen_kv((4, 4, 131072, 128), 21)
    bits, scales, rot = H.encode_tiles(x, T, O.DCT, want_rotated=True)
    torch.cuda.synchronize()
    for s in (3, 14):
        xs = x.view(16, 131072, 128)[s, :16384].float().cpu().numpy()  # first 128 tiles
        rs_gpu = rot.view(16, 131072, 128)[s, :16384].cpu().numpy()
        ref = xs.astype(np.float64) @ O.dct_matrix().T
        err = np.abs(rs_gpu - ref).max(axis=-1) / np.maximum(np.linalg.norm(xs, axis=-1), 1e-30)
        assert err.max() < 1e-6, (s, err.max())
        rb, rsc = O.encode_tiles(rs_gpu[None], T)
        gb = bits.view(16, -1)[s].cpu().numpy().view(np.uint64).reshape(1, -1)[:, :rb.size].reshape(rb.shape)
        assert np.array_equal(gb, rb), s
        assert np.array_equal(scales[s, :128].cpu().numpy().view(np.uint16), rsc.view(np.uint16).reshape(-1)), s
