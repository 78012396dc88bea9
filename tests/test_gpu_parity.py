"""GPU parity of every HIP kernel against the CPU oracle, called through the C ABI.

Bar: packed bits and tile scales bit-exact given the same
fp32 rotated input; tile scores and top-k bit/index-exact (scores follow a fixed fp32
order the oracle emulates, so there are no tie ambiguities); attention within 1e-5
max-abs for fp32 output and within 2e-3 + bf16 rounding (2^-8 |ref|) for bf16 output,
both against a float64 reference on the same stored inputs.
"""
import numpy as np
import pytest
import torch

from conftest import kv_like
from oracle import kvr_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
TDT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def H():
    from modules import _hip
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    _hip.lib()
    return _hip


def u64(t):
    return t.cpu().numpy().view(np.uint64)


def f16bits(t):
    return t.cpu().numpy().view(np.uint16)


def f32bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ----------------------------------------------------------------------------- encoder

@pytest.mark.parametrize("T", [64, 128])
@pytest.mark.parametrize("dt", ["bf16", "fp16", "fp32"])
def test_encode_hadamard_bit_exact(H, rng, T, dt):
    say(f"[encode/hadamard] T={T} dtype={dt}")
    n_b, n_h, n_tok = 2, 3, 3 * T
    xt = torch.from_numpy(kv_like(rng, (n_b, n_h, n_tok, 128))).to(DEV, TDT[dt])
    xv = xt.float().cpu().numpy().reshape(n_b * n_h, n_tok, 128)
    bits, scales, rot = H.encode_tiles(xt, T, H.HADAMARD, want_rotated=True)
    torch.cuda.synchronize()
    ref_rot = O.hadamard_rotate(xv)
    assert np.array_equal(f32bits(rot.cpu().numpy()), f32bits(ref_rot)), "rotation not bit-exact"
    rb, rs = O.encode_tiles(ref_rot, T)
    assert np.array_equal(u64(bits), rb)
    assert np.array_equal(f16bits(scales), rs.view(np.uint16))


@pytest.mark.parametrize("T", [64, 128])
def test_encode_dct_codec_exact_given_rotation(H, rng, T):
    say(f"[encode/dct] T={T}")
    xt = torch.from_numpy(kv_like(rng, (1, 2, 2 * T, 128))).to(DEV, torch.bfloat16)
    xv = xt.float().cpu().numpy().reshape(2, 2 * T, 128)
    bits, scales, rot = H.encode_tiles(xt, T, H.DCT, want_rotated=True)
    torch.cuda.synchronize()
    rot = rot.cpu().numpy()
    ref = xv.astype(np.float64) @ O.dct_matrix().T
    err = np.abs(rot - ref).max(axis=-1) / np.linalg.norm(xv, axis=-1)
    assert err.max() < 1e-6, err.max()
    rb, rs = O.encode_tiles(rot, T)  # codec bit-exact given the kernel's own rotation
    assert np.array_equal(u64(bits), rb)
    assert np.array_equal(f16bits(scales), rs.view(np.uint16))


@pytest.mark.parametrize("T", [64, 128])
def test_encode_prerotated_fp32(H, rng, T):
    say(f"[encode/none] T={T}")
    y = kv_like(rng, (1, 4, 2 * T, 128))
    bits, scales = H.encode_tiles(torch.from_numpy(y).to(DEV), T, H.NONE)
    rb, rs = O.encode_tiles(y.reshape(4, 2 * T, 128), T)
    assert np.array_equal(u64(bits), rb)
    assert np.array_equal(f16bits(scales), rs.view(np.uint16))


def test_encode_strided_token_major_into_offset_slots(H, rng):
    say("[encode/strided] [B, N, Hkv, d] view into tile slots 3..5 of a 9-slot store")
    T, B, N, Hkv = 64, 2, 192, 4
    full = torch.from_numpy(kv_like(rng, (B, N, Hkv, 128))).to(DEV, torch.bfloat16)
    view = full.permute(0, 2, 1, 3)  # [B, Hkv, N, d], token stride Hkv*d
    bits, scales = H.alloc_store(B * Hkv, 9, T, DEV)
    H.encode_tiles(view, T, H.HADAMARD, bits=bits, scales=scales, tile_offset=3)
    xv = view.float().cpu().numpy().reshape(B * Hkv, N, 128)
    rb, rs = O.encode(xv, T, O.HADAMARD)
    gb, gs = u64(bits), f16bits(scales)
    assert np.array_equal(gb[:, 3:6], rb)
    assert np.array_equal(gs[:, 3:6], rs.view(np.uint16))
    assert not gb[:, :3].any() and not gb[:, 6:].any(), "wrote outside its tile slots"


def test_encode_edge_tiles(H):
    say("[encode/edges] zero tile, constant tile, fp16-saturating tile")
    T = 64
    x = np.zeros((1, 3, T, 128), np.float32)
    x[0, 1] = 0.37
    x[0, 2] = 1.0e7   # mean |y| = 1e7/sqrt(128) > fp16 max
    xt = torch.from_numpy(x).to(DEV, torch.bfloat16)
    bits, scales, rot = H.encode_tiles(xt, T, H.HADAMARD, want_rotated=True)
    torch.cuda.synchronize()
    rb, rs = O.encode_tiles(rot.cpu().numpy(), T)
    assert np.array_equal(u64(bits), rb)
    assert np.array_equal(f16bits(scales), rs.view(np.uint16))
    s = scales.cpu().numpy().astype(np.float32)[:, 0]
    assert s[0] == 0 and np.all(u64(bits)[0] == np.uint64(0xFFFFFFFFFFFFFFFF))  # u = +0 -> bit 1
    assert s[2] == 65504.0


def test_encode_deterministic(H, rng):
    say("[encode/determinism] two runs, same bits")
    xt = torch.from_numpy(kv_like(rng, (4, 8, 512, 128))).to(DEV, torch.bfloat16)
    a = H.encode_tiles(xt, 64, H.HADAMARD)
    b = H.encode_tiles(xt, 64, H.HADAMARD)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("T,tf,dt", [(64, "had", "bf16"), (64, "had", "fp32"), (128, "had", "bf16"),
                                     (64, "dct", "bf16"), (128, "dct", "bf16"), (128, "dct", "fp32"),
                                     (64, "none", "fp32")])
def test_encode_counts_are_channel_popcounts(H, rng, T, tf, dt):
    """The per-tile channel counts every encoder kernel writes next to the bits equal the
    number of set bits of each channel word (summed over a T=128 tile's two words), in the
    same tile slots; slots outside the encoded range stay untouched."""
    say(f"[encode/counts] T={T} tf={tf} dtype={dt}")
    tfv = {"had": H.HADAMARD, "dct": H.DCT, "none": H.NONE}[tf]
    n_b, n_h, n_tok = 2, 3, 5 * T
    xt = torch.from_numpy(kv_like(rng, (n_b, n_h, n_tok, 128))).to(DEV, TDT[dt])
    bits, scales = H.alloc_store(n_b * n_h, 7, T, DEV)
    counts = H.alloc_counts(n_b * n_h, 7, DEV)
    H.encode_tiles(xt, T, tfv, bits=bits, scales=scales, tile_offset=1, counts=counts)
    b = u64(bits)  # [seg, tile, 128, T/64]
    pc = np.unpackbits(b.view(np.uint8), axis=-1).reshape(b.shape + (64,)).sum(axis=(-1, -2))
    c = counts.cpu().numpy()
    assert np.array_equal(c[:, 1:6], pc[:, 1:6].astype(np.uint8))
    assert not c[:, 0].any() and not c[:, 6].any(), "wrote outside its tile slots"


# ----------------------------------------------------------------------------- query prep

@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (28, 4), (8, 8)])
@pytest.mark.parametrize("dt", ["bf16", "fp32"])
def test_query_prep_hadamard_bit_exact(H, rng, Hq, Hkv, dt):
    say(f"[query_prep] Hq={Hq} Hkv={Hkv} dt={dt}")
    q = torch.from_numpy(rng.standard_normal((3, Hq, 128)).astype(np.float32)).to(DEV, TDT[dt])
    qbar, qrot = H.query_prep(q, Hkv, H.HADAMARD)
    rb, rr = O.query_prep(q.float().cpu().numpy(), Hkv, O.HADAMARD)
    assert np.array_equal(f32bits(qbar.cpu().numpy()), f32bits(rb.reshape(-1, 128)))
    assert np.array_equal(f32bits(qrot.cpu().numpy()), f32bits(rr.reshape(-1, 128)))


def test_query_prep_dct(H, rng):
    say("[query_prep/dct]")
    q = torch.from_numpy(rng.standard_normal((2, 28, 128)).astype(np.float32)).to(DEV)
    qbar, qrot = H.query_prep(q, 4, H.DCT)
    mean = O.gqa_mean(q.cpu().numpy(), 4).astype(np.float64)
    ref = mean @ O.dct_matrix().T
    assert np.abs(qbar.cpu().numpy().reshape(2, 4, 128) - ref).max() < 1e-5
    ref_r = q.cpu().numpy().astype(np.float64) @ O.dct_matrix().T
    assert np.abs(qrot.cpu().numpy().reshape(2, 28, 128) - ref_r).max() < 1e-5


# ----------------------------------------------------------------------------- scoring

def random_bits(rng, shape):
    return rng.integers(0, 2 ** 63, size=shape, dtype=np.int64).view(np.uint64) ^ \
        (rng.integers(0, 2, size=shape, dtype=np.int64).astype(np.uint64) << np.uint64(63))


@pytest.mark.parametrize("T", [64, 128])
@pytest.mark.parametrize("method", [0, 1])
def test_score_bit_exact(H, rng, T, method):
    say(f"[score] T={T} method={method}")
    S, n_tiles, cap = 6, 203, 211
    bits = random_bits(rng, (S, cap, 128, T // 64))
    # bias some tiles so scores spread (not all near 0)
    bits[:, ::7] |= np.uint64(0xFFFF0000FFFF0000)
    qbar = rng.standard_normal((S, 128)).astype(np.float32)
    lo = np.array([0, 5, 0, 100, 202, 0], np.int32)
    hi = np.array([0, 9, 300, 101, 203, 1], np.int32)
    tb = torch.from_numpy(bits.view(np.int64)).to(DEV)
    sc = H.score_tiles(torch.from_numpy(qbar).to(DEV), tb, n_tiles, T,
                       excl_lo=torch.from_numpy(lo).to(DEV), excl_hi=torch.from_numpy(hi).to(DEV),
                       method=method)
    ref = O.score_tiles(qbar, bits[:, :n_tiles], excl=(lo, hi))
    assert np.array_equal(f32bits(sc.cpu().numpy()), f32bits(ref))


def test_score_nan_query_is_minus_inf(H, rng):
    say("[score/nan]")
    bits = random_bits(rng, (2, 8, 128, 1))
    q = rng.standard_normal((2, 128)).astype(np.float32)
    q[1, 5] = np.nan
    sc = H.score_tiles(torch.from_numpy(q).to(DEV), torch.from_numpy(bits.view(np.int64)).to(DEV), 8, 64)
    s = sc.cpu().numpy()
    assert np.all(np.isneginf(s[1])) and np.all(np.isfinite(s[0]))


# ----------------------------------------------------------------------------- top-k

@pytest.mark.parametrize("n,k", [(496, 32), (1008, 64), (56, 8), (37, 37), (300, 1), (2500, 1024)])
def test_topk_exact(H, rng, n, k):
    say(f"[topk] n={n} k={k}")
    S = 5
    s = rng.standard_normal((S, n)).astype(np.float32)
    s[1] = np.round(s[1] * 4) / 4                     # heavy ties
    s[2, ::3] = -np.inf                                # excluded tiles
    s[3, 5:20] = np.nan                                # NaN -> -inf
    s[4] = 0.5                                         # all equal
    idx = H.topk_tiles(torch.from_numpy(s).to(DEV), k)
    assert np.array_equal(idx.cpu().numpy(), O.topk_tiles(s, k))


# ----------------------------------------------------------------------------- attention

def make_store(rng, S, n_tiles, T):
    kb = random_bits(rng, (S, n_tiles, 128, T // 64))
    vb = random_bits(rng, (S, n_tiles, 128, T // 64))
    ks = (0.5 + rng.random((S, n_tiles))).astype(np.float16)
    vs = (0.5 + rng.random((S, n_tiles))).astype(np.float16)
    return kb, vb, ks, vs


def dev_store(kb, vb, ks, vs):
    return (torch.from_numpy(kb.view(np.int64)).to(DEV), torch.from_numpy(vb.view(np.int64)).to(DEV),
            torch.from_numpy(ks).to(DEV), torch.from_numpy(vs).to(DEV))


def check_out(out, ref, what):
    o = out.float().cpu().numpy()
    if out.dtype == torch.float32:
        err = np.abs(o - ref).max()
        assert err <= 1e-5, f"{what}: fp32 max-abs {err}"
    else:
        excess = (np.abs(o - ref) - (2e-3 + np.abs(ref) * 2.0 ** -8)).max()
        assert excess <= 0, f"{what}: bf16 error exceeds 2e-3 + 2^-8|ref| by {excess}"


ATTN_CASES = [
    # B, Hq, Hkv, win_len, W_cap, n_tiles, k, T, tf, qdt, wdt
    (2, 32, 8, 96, 128, 10, 3, 64, O.HADAMARD, "bf16", "bf16"),
    (1, 28, 4, 300, 320, 9, 2, 128, O.DCT, "bf16", "bf16"),
    (2, 8, 8, 33, 64, 5, 5, 64, O.HADAMARD, "fp32", "bf16"),
    (1, 32, 8, 512, 512, 56, 8, 64, O.HADAMARD, "fp32", "bf16"),
    (2, 16, 2, 64, 64, 4, 0, 64, O.HADAMARD, "bf16", "fp16"),
    (2, 12, 4, 0, 64, 6, 4, 64, O.HADAMARD, "fp16", "fp16"),
    (1, 64, 4, 40, 64, 6, 2, 128, O.DCT, "fp32", "fp16"),
    (1, 32, 8, 256, 256, 80, 37, 64, O.HADAMARD, "bf16", "bf16"),
]


@pytest.fixture(params=["mfma", "valu"])
def ret_method(request, monkeypatch):
    """Both arithmetic paths of the retrieved tiles (read by the library at every launch)."""
    monkeypatch.setenv("KVR_RETRIEVE_METHOD", request.param)
    return request.param


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_w{}_k{}_T{}_tf{}_{}_{}".format(
    c[0], c[1], c[2], c[3], c[6], c[7], c[8], c[9], c[10]))
@pytest.mark.parametrize("odt", ["fp32", "bf16"])
def test_decode_attn(H, rng, case, odt, ret_method):
    B, Hq, Hkv, wl, wcap, n_tiles, k, T, tf, qdt, wdt = case
    say(f"[decode_attn] {case} out={odt} retrieve={ret_method}")
    S = B * Hkv
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, TDT[qdt])
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, wcap, 128))).to(DEV, TDT[wdt])
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, wcap, 128)).astype(np.float32)).to(DEV, TDT[wdt])
    kb, vb, ks, vs = make_store(rng, S, n_tiles, T)
    idx = np.stack([rng.permutation(n_tiles)[:k] for _ in range(S)]).astype(np.int32).reshape(S, k)
    tkb, tvb, tks, tvs = dev_store(kb, vb, ks, vs)
    out = H.decode_attn(q, wk, wv, wl, tkb, tvb, tks, tvs, torch.from_numpy(idx).to(DEV) if k else None,
                        T, tf, out_dtype=TDT[odt])
    torch.cuda.synchronize()
    ref = O.decode_attention(q.float().cpu().numpy(), wk.float().cpu().numpy(), wv.float().cpu().numpy(),
                             kb, vb, ks, vs, idx, tf, win_len=wl)
    check_out(out, ref, str(case))


def test_decode_attn_window_token_major_strides(H, rng):
    say("[decode_attn/strides] window stored [B, W, Hkv, d]")
    B, Hq, Hkv, W, T = 2, 32, 8, 200, 64
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    wk_tm = torch.from_numpy(kv_like(rng, (B, W, Hkv, 128))).to(DEV, torch.bfloat16)
    wv_tm = torch.from_numpy(rng.standard_normal((B, W, Hkv, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    wk, wv = wk_tm.permute(0, 2, 1, 3), wv_tm.permute(0, 2, 1, 3)
    kb, vb, ks, vs = make_store(rng, B * Hkv, 7, T)
    idx = np.stack([rng.permutation(7)[:3] for _ in range(B * Hkv)]).astype(np.int32)
    out = H.decode_attn(q, wk, wv, W, *dev_store(kb, vb, ks, vs), torch.from_numpy(idx).to(DEV), T,
                        H.HADAMARD, out_dtype=torch.float32)
    ref = O.decode_attention(q.float().cpu().numpy(), wk.float().cpu().numpy(), wv.float().cpu().numpy(),
                             kb, vb, ks, vs, idx, O.HADAMARD)
    check_out(out, ref, "token-major window")


def test_decode_attn_peaked_softmax(H, rng, ret_method):
    say(f"[decode_attn/peaked] one dominant window key and one dominant retrieved tile ({ret_method})")
    B, Hq, Hkv, W, T = 1, 8, 2, 64, 64
    qn = rng.standard_normal((B, Hq, 128)).astype(np.float32)
    wkn = 0.1 * rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)
    wkn[0, 0, 17] = 4.0 * qn[0, 0]
    q = torch.from_numpy(qn).to(DEV, torch.bfloat16)
    wk = torch.from_numpy(wkn).to(DEV, torch.bfloat16)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    kb, vb, ks, vs = make_store(rng, B * Hkv, 4, T)
    idx = np.array([[0, 1], [2, 3]], np.int32)
    for odt in (torch.float32, torch.bfloat16):
        out = H.decode_attn(q, wk, wv, W, *dev_store(kb, vb, ks, vs), torch.from_numpy(idx).to(DEV), T,
                            H.HADAMARD, out_dtype=odt)
        ref = O.decode_attention(q.float().cpu().numpy(), wk.float().cpu().numpy(), wv.float().cpu().numpy(),
                                 kb, vb, ks, vs, idx, O.HADAMARD)
        check_out(out, ref, "peaked")


# ----------------------------------------------------------------------------- full step

@pytest.mark.parametrize("tf,T,Hq,Hkv", [(O.HADAMARD, 64, 32, 8), (O.DCT, 128, 28, 4)])
def test_decode_step_matches_oracle_pipeline(H, rng, tf, T, Hq, Hkv, ret_method):
    say(f"[decode_step] tf={tf} T={T} Hq={Hq} Hkv={Hkv} retrieve={ret_method}")
    B, W, n_tok, k = 2, 256, 40 * T, 6
    K = torch.from_numpy(kv_like(rng, (B, Hkv, n_tok, 128))).to(DEV, torch.bfloat16)
    V = torch.from_numpy(rng.standard_normal((B, Hkv, n_tok, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    kb, ks = H.encode_tiles(K, T, tf)
    vb, vs = H.encode_tiles(V, T, tf)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, W, 128))).to(DEV, torch.bfloat16)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    n_tiles = n_tok // T
    lo_np = np.zeros(B * Hkv, np.int32)
    hi_np = np.zeros(B * Hkv, np.int32)
    lo_np[1], hi_np[1] = 3, 5          # exclude tiles 3..4 of segment 1
    lo_np[-1], hi_np[-1] = 0, 1        # and tile 0 of the last segment
    lo = torch.from_numpy(lo_np).to(DEV)
    hi = torch.from_numpy(hi_np).to(DEV)
    idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
    out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, excl_lo=lo, excl_hi=hi,
                        out_dtype=torch.float32, idx_out=idx)
    torch.cuda.synchronize()
    kbn, vbn, ksn, vsn = u64(kb), u64(vb), ks.cpu().numpy(), vs.cpu().numpy()
    qn = q.float().cpu().numpy()
    qbar_ref, _ = O.query_prep(qn, Hkv, tf)
    sref = O.score_tiles(qbar_ref.reshape(-1, 128), kbn, excl=(lo.cpu().numpy(), hi.cpu().numpy()))
    iref = O.topk_tiles(sref, k)
    ig = idx.cpu().numpy()
    if tf == O.HADAMARD:
        assert np.array_equal(ig, iref)
    else:  # DCT query rotation is a tolerance: identical up to near-ties of the k-th score
        for s in range(ig.shape[0]):
            if not np.array_equal(np.sort(ig[s]), np.sort(iref[s])):
                kth = np.sort(sref[s])[::-1][k - 1]
                diff = set(ig[s]) ^ set(iref[s])
                assert all(abs(sref[s][t] - kth) <= 1e-6 * np.abs(sref[s]).max() for t in diff)
    ref = O.decode_attention(qn, wk.float().cpu().numpy(), wv.float().cpu().numpy(), kbn, vbn, ksn, vsn, ig, tf)
    check_out(out, ref, "decode_step")


@pytest.mark.parametrize("tf,T,Hq,Hkv", [(O.HADAMARD, 64, 32, 8), (O.DCT, 128, 28, 4)])
def test_decode_step_counts_equal_bits(H, rng, tf, T, Hq, Hkv):
    """Scoring from the per-tile channel counts gives the same step bit for bit: the same
    selected tiles and the same output as scoring from the K bits (with an exclusion)."""
    say(f"[decode_step/counts] tf={tf} T={T}")
    B, W, n_tok, k = 3, 192, 50 * T, 7
    K = torch.from_numpy(kv_like(rng, (B, Hkv, n_tok, 128))).to(DEV, torch.bfloat16)
    V = torch.from_numpy(rng.standard_normal((B, Hkv, n_tok, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    counts = H.alloc_counts(B * Hkv, n_tok // T, DEV)
    kb, ks = H.encode_tiles(K, T, tf, counts=counts)
    vb, vs = H.encode_tiles(V, T, tf)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, W, 128))).to(DEV, torch.bfloat16)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    lo = torch.zeros(B * Hkv, dtype=torch.int32, device=DEV)
    hi = torch.zeros(B * Hkv, dtype=torch.int32, device=DEV)
    lo[2], hi[2] = 4, 9
    res = []
    for kc in (None, counts):
        idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
        out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tok // T, T, tf, k, excl_lo=lo, excl_hi=hi,
                            out_dtype=torch.float32, idx_out=idx, kcounts=kc)
        torch.cuda.synchronize()
        res.append((idx.cpu().numpy(), out.cpu().numpy()))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1].view(np.uint32), res[1][1].view(np.uint32))


def test_decode_step_workspace_reuse(H, rng):
    """One workspace across calls of different shapes: after every call the error word and
    the records-done counters are zero (the per-segment epochs advance), and repeated calls
    give bit-identical outputs (the merge order is fixed)."""
    say("[decode_step/workspace reuse] counters settle; repeat calls bit-identical")
    T, tf = 64, O.HADAMARD
    ws = H.decode_step_workspace(4, 32, 8, 512, 64, 16, T, DEV)
    outs = []
    for B, Hkv, n_tiles, k, W in [(2, 8, 40, 6, 256), (4, 8, 64, 16, 512), (2, 8, 40, 6, 256), (1, 4, 33, 33, 0)]:
        Hq = 4 * Hkv
        gen = np.random.default_rng(7 + B + n_tiles)
        K = torch.from_numpy(kv_like(gen, (B, Hkv, n_tiles * T, 128))).to(DEV, torch.bfloat16)
        V = torch.from_numpy(gen.standard_normal((B, Hkv, n_tiles * T, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
        kb, ks = H.encode_tiles(K, T, tf)
        vb, vs = H.encode_tiles(V, T, tf)
        q = torch.from_numpy(gen.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
        wk = torch.from_numpy(kv_like(gen, (B, Hkv, max(W, 1), 128))).to(DEV, torch.bfloat16)
        wv = torch.from_numpy(gen.standard_normal((B, Hkv, max(W, 1), 128)).astype(np.float32)).to(DEV, torch.bfloat16)
        assert ws.numel() >= H.lib().kvr_decode_step_workspace(B, Hq, Hkv, W, n_tiles, k, T)
        o1 = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=torch.float32, workspace=ws)
        o2 = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
        ctr = ws[:H.COUNTER_BYTES].view(torch.int32)
        assert int(ctr[0].item()) == 0, "a bounded wait gave up"                      # error word
        assert int(ctr[64 + 4096 * 32:].count_nonzero().item()) == 0                    # records-done lines
        ig = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
        H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=torch.float32, idx_out=ig,
                      workspace=ws)
        qn = q.float().cpu().numpy()
        ref = O.decode_attention(qn, wk.float().cpu().numpy()[:, :, :W], wv.float().cpu().numpy()[:, :, :W],
                                 u64(kb), u64(vb), ks.cpu().numpy(), vs.cpu().numpy(), ig.cpu().numpy(), tf)
        check_out(o1, ref, f"reuse B={B} n_tiles={n_tiles} k={k} W={W}")
        outs.append(o1)
    assert torch.equal(outs[0], outs[2])


def test_decode_step_window_only(H, rng):
    say("[decode_step/window-only] n_tiles = 0")
    B, Hq, Hkv, W = 2, 32, 8, 100
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, W, 128))).to(DEV, torch.bfloat16)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    out = H.decode_step(q, wk, wv, W, None, None, None, None, 0, 64, H.HADAMARD, 0, out_dtype=torch.float32)
    ref = O.decode_attention(q.float().cpu().numpy(), wk.float().cpu().numpy(), wv.float().cpu().numpy(),
                             None, None, None, None, None, O.HADAMARD)
    check_out(out, ref, "window only")
    sdpa = torch.nn.functional.scaled_dot_product_attention(
        q.float().view(B, Hkv, Hq // Hkv, 128), wk.float(), wv.float())
    assert (out.view(B, Hkv, Hq // Hkv, 128) - sdpa).abs().max().item() < 1e-5


# ----------------------------------------------------------------------------- gather

@pytest.mark.parametrize("T,tf", [(64, O.HADAMARD), (128, O.DCT), (64, O.NONE)])
def test_gather_tiles(H, rng, T, tf):
    say(f"[gather] T={T} tf={tf}")
    S, n = 3, 9
    kb, _, ks, _ = make_store(rng, S, n, T)
    idx = np.stack([rng.permutation(n)[:4] for _ in range(S)]).astype(np.int32)
    out = H.gather_tiles(torch.from_numpy(kb.view(np.int64)).to(DEV), torch.from_numpy(ks).to(DEV),
                         torch.from_numpy(idx).to(DEV), T, tf)
    ref = np.stack([O.dequantize_original(kb[s][idx[s]], ks[s][idx[s]], tf).reshape(-1, 128) for s in range(S)])
    assert np.abs(out.cpu().numpy() - ref).max() < 2e-6 * max(1.0, np.abs(ref).max())
