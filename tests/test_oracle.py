"""Pins the CPU oracle independently of its own formulas (CPU only).

Each check is chosen so a plausible mistake (dropped term, wrong sign/index, transposed
operand, wrong stage order of the exclusion arithmetic) fails it: closed forms, library
routines (scipy, torch, transformers), brute force, hand-computed known answers, and
exact identities of the sigma-delta recurrence.
"""
import numpy as np
import pytest
import scipy.fft
import scipy.linalg
import torch

from conftest import kv_like
from oracle import kvr_oracle as O


# ----------------------------------------------------------------------------- transforms

def test_fwht_hand_kat():
    assert np.array_equal(O.fwht(np.array([1, 2, 3, 4], np.float32)), [10, -2, -4, 0])
    e0 = np.zeros(128, np.float32)
    e0[0] = 1
    assert np.array_equal(O.fwht(e0), np.ones(128, np.float32))


@pytest.mark.parametrize("n", [2, 4, 8, 128])
def test_fwht_is_sylvester_hadamard(n, rng):
    x = rng.standard_normal((5, n))
    assert np.allclose(O.fwht(x, np.float64), x @ scipy.linalg.hadamard(n).T, atol=1e-12)


def test_hadamard_rotation_orthonormal_and_fp32_close(rng):
    Hm = scipy.linalg.hadamard(128) / np.sqrt(128)
    assert np.allclose(Hm @ Hm.T, np.eye(128), atol=1e-12)
    x = kv_like(rng, (50, 128))
    y = O.hadamard_rotate(x).astype(np.float64)
    ref = x.astype(np.float64) @ Hm.T
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-6
    assert np.allclose(O.inverse_rotate64(O.rotate64(x, O.HADAMARD), O.HADAMARD), x, atol=1e-5)
    assert O.C_HAD == np.float32(2 ** -3.5)


def test_dct_matches_scipy_and_is_orthonormal(rng):
    C = O.dct_matrix()
    assert np.allclose(C, scipy.fft.dct(np.eye(128), type=2, norm="ortho", axis=0), atol=1e-13)
    assert np.allclose(C @ C.T, np.eye(128), atol=1e-13)
    x = rng.standard_normal((4, 128))
    assert np.allclose(O.rotate64(x, O.DCT), scipy.fft.dct(x, norm="ortho", axis=-1), atol=1e-12)
    assert np.allclose(O.inverse_rotate64(O.rotate64(x, O.DCT), O.DCT), x, atol=1e-12)


# ----------------------------------------------------------------------------- scale

def test_tile_scale_kats():
    y = np.ones((64, 128), np.float32)
    assert O.tile_scale(y) == np.float16(1.0)
    y = np.zeros((64, 128), np.float32)
    y[:, ::2] = -0.5
    assert O.tile_scale(y) == np.float16(0.25)
    assert O.tile_scale(np.zeros((128, 128), np.float32)) == np.float16(0.0)
    assert O.tile_scale(np.full((64, 128), 1e6, np.float32)) == np.float16(65504.0)


def test_tile_scale_close_to_float64_mean(rng):
    y = kv_like(rng, (20, 64, 128))
    s = O.tile_scale(y).astype(np.float64)
    m = np.abs(y.astype(np.float64)).mean(axis=(1, 2))
    assert np.all(np.abs(s - m) <= m * 2.0 ** -10)


# ----------------------------------------------------------------------------- sigma-delta

def sd_scalar(y, s):
    """Independent scalar restatement with explicit float32 scalars: bits and final error."""
    s = np.float32(s)
    e = np.float32(0.0)
    bits = []
    for v in y:
        u = np.float32(np.float32(v) + e)
        b = 1 if u >= 0 else 0
        q = s if b else np.float32(-s)
        e = np.float32(u - q)
        bits.append(b)
    return bits, e


@pytest.mark.parametrize("T", [64, 128])
def test_sigma_delta_matches_scalar_loop_and_tile_sum_identity(rng, T):
    y = kv_like(rng, (3, T, 128))
    s = O.tile_scale(y)
    words = O.sigma_delta_pack(y, s)
    b = O.unpack_bits(words)
    for i in range(3):
        for ch in (0, 5, 77, 127):
            bits, eT = sd_scalar(y[i, :, ch], s[i].astype(np.float32))
            assert list(b[i, :, ch]) == bits
            q = np.float64(s[i]) * (2.0 * np.array(bits) - 1.0)
            # sum_t q_t = sum_t y_t + e_0 - e_T  (exact in reals; fp32 rounding of u and e only)
            resid = q.sum() - y[i, :, ch].astype(np.float64).sum() + np.float64(eT)
            assert abs(resid) <= 1e-5 * (np.abs(y[i, :, ch]).sum() + s[i])


def test_sigma_delta_error_bounded_by_scale_for_bounded_input(rng):
    c = np.float32(0.75)  # exactly representable in fp16, so s == |y|
    y = (c * np.sign(rng.standard_normal((4, 64, 128)) + 1e-9)).astype(np.float32)
    s = O.tile_scale(y)
    assert np.all(s == np.float16(0.75))
    q = O.dequantize(O.sigma_delta_pack(y, s), s)
    assert np.all(np.abs(q.sum(axis=-2) - y.astype(np.float64).sum(axis=-2)) <= 0.75 + 1e-6)


def test_sigma_delta_kat_words():
    s = np.float16(1.0)
    alt = np.tile(np.array([1.0, -1.0], np.float32), 32)[:, None].repeat(128, 1)
    assert np.all(O.sigma_delta_pack(alt, s) == np.uint64(0x5555555555555555))
    half = np.full((64, 128), 0.5, np.float32)   # 1,1,0,1 repeating -> 0xB per nibble
    assert np.all(O.sigma_delta_pack(half, s) == np.uint64(0xBBBBBBBBBBBBBBBB))
    zero = np.zeros((64, 128), np.float32)       # u = +0 -> 1, then -1 -> 0
    assert np.all(O.sigma_delta_pack(zero, s) == np.uint64(0x5555555555555555))


@pytest.mark.parametrize("c", [-0.6, -0.1, 0.0, 0.3, 0.9])
def test_sigma_delta_constant_input_density(c):
    y = np.full((128, 128), c, np.float32)
    b = O.unpack_bits(O.sigma_delta_pack(y, np.float16(1.0)))
    assert abs(b.mean() - (c + 1) / 2) <= 1.0 / 128 + 1e-12


def test_pack_unpack_roundtrip_and_layout(rng):
    b = rng.integers(0, 2, size=(3, 128, 128), dtype=np.uint8)
    w = O.pack_bits(b)
    assert w.shape == (3, 128, 2)
    assert np.array_equal(O.unpack_bits(w), b)
    one = np.zeros((64, 128), np.uint8)
    one[5, 3] = 1           # token 5 of channel 3
    one[63, 127] = 1        # last token of the last channel
    w = O.pack_bits(one)
    assert w[3, 0] == np.uint64(1 << 5) and w[127, 0] == np.uint64(1 << 63)
    assert np.count_nonzero(w) == 2


# ----------------------------------------------------------------------------- scoring

def random_words(rng, shape):
    return rng.integers(0, 2 ** 63, size=shape, dtype=np.int64).view(np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=shape, dtype=np.int64).astype(np.uint64)


@pytest.mark.parametrize("T", [64, 128])
def test_scores_match_bruteforce_and_reference_definition(rng, T):
    bits = random_words(rng, (4, 30, 128, T // 64))
    bits[:, ::5] |= np.uint64(0x00FF00FF00FF00FF)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    s = O.score_tiles(q, bits)
    bf = O.score_tiles_bruteforce(q, bits)
    assert np.abs(s - bf).max() <= 1e-6
    scales = (0.2 + rng.random((4, 30))).astype(np.float16)
    assert np.abs(s - O.score_tiles_reference_def(q, bits, scales)).max() <= 1e-5


def test_score_special_cases(rng):
    bits = random_words(rng, (2, 6, 128, 1))
    bits[0, 2] = np.uint64(0x00000000FFFFFFFF)   # every column sum 0 -> score 0
    q = rng.standard_normal((2, 128)).astype(np.float32)
    q[1, 0] = np.nan
    s = O.score_tiles(q, bits, excl=(np.array([4, 0]), np.array([6, 0])))
    assert s[0, 2] == 0.0
    assert np.all(np.isneginf(s[0, 4:6])) and np.all(np.isfinite(s[0, :4]))
    assert np.all(np.isneginf(s[1]))


def test_exclusion_and_k_rule_hand_cases():
    # modules/kvr_retrieval.py:373-378, computed by hand
    assert O.exclusion_to_tiles(0, 0, 64, 10) == (0, 0)
    assert O.exclusion_to_tiles(70, 130, 64, 10) == (1, 3)
    assert O.exclusion_to_tiles(0, 640, 64, 10) == (0, 10)
    assert O.exclusion_to_tiles(600, 700, 64, 10) == (9, 10)
    assert O.exclusion_to_tiles(128, 128, 64, 10) == (0, 0)
    assert O.k_tiles(128, 64, 10) == 2
    assert O.k_tiles(10, 64, 10) == 1
    assert O.k_tiles(1000, 64, 5) == 5


def test_topk_bruteforce(rng):
    for trial in range(20):
        n = int(rng.integers(1, 60))
        k = int(rng.integers(1, n + 1))
        s = np.round(rng.standard_normal((2, n)) * 2).astype(np.float32) / 2
        s[1, rng.integers(0, n)] = -np.inf
        got = O.topk_tiles(s, k)
        for r in range(2):
            want = sorted(range(n), key=lambda i: (-float(s[r, i]), i))[:k]
            assert list(got[r]) == want


def test_topk_nan_is_minus_inf():
    s = np.array([[np.nan, 1.0, -np.inf, 0.0]], np.float32)
    assert list(O.topk_tiles(s, 4)[0]) == [1, 3, 0, 2]


# ----------------------------------------------------------------------------- query side

@pytest.mark.parametrize("g", [1, 4, 7])
def test_gqa_mean_matches_torch(rng, g):
    q = rng.standard_normal((2, 4 * g, 128)).astype(np.float32)
    ref = torch.from_numpy(q).view(2, 4, g, 128).mean(2).numpy()
    got = O.gqa_mean(q, 4)
    if g in (1, 4):
        assert np.array_equal(got, ref)
    else:
        assert np.abs(got - ref).max() <= 2 * np.spacing(np.abs(ref).max())


def test_rope_matches_transformers(rng):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, rope_theta=500000.0,
                      max_position_embeddings=8192)
    emb = LlamaRotaryEmbedding(cfg)
    x = torch.zeros(1, 100, 128)
    cos0, sin0 = emb(x, torch.arange(0, 100)[None])
    c0, s0 = O.rope_tables(100, base=500000.0)
    assert np.abs(cos0[0].numpy() - c0).max() < 1e-4 and np.abs(sin0[0].numpy() - s0).max() < 1e-4
    pos = torch.arange(3000, 3100)[None]
    cos, sin = emb(x, pos)
    c, s = O.rope_tables(100, base=500000.0, start=3000)
    # fp32 angles pos*inv_freq differ by at most ~2 ulp between implementations
    tol = 4 * 3100 * 2.0 ** -24 + 1e-6
    assert np.abs(cos[0].numpy() - c).max() < tol and np.abs(sin[0].numpy() - s).max() < tol
    k = rng.standard_normal((1, 8, 100, 128)).astype(np.float32)
    _, k_hf = apply_rotary_pos_emb(torch.from_numpy(k), torch.from_numpy(k), cos, sin)
    ch, sh = cos[0].numpy()[None, None], sin[0].numpy()[None, None]
    k_or = O.apply_rotary(k, ch, sh)          # same tables: pins the rotate_half convention
    assert np.abs(k_hf.numpy() - k_or).max() < 1e-5
    assert np.allclose(O.reverse_rotary(k_or, ch, sh), k, atol=1e-4)


# ----------------------------------------------------------------------------- attention

@pytest.mark.parametrize("tf", [O.HADAMARD, O.DCT])
def test_attention_oracle_matches_sdpa_on_dequantised_tokens(rng, tf):
    B, Hq, Hkv, W, T, n, k = 2, 8, 2, 40, 64, 5, 2
    q = rng.standard_normal((B, Hq, 128)).astype(np.float32)
    wk = kv_like(rng, (B, Hkv, W, 128))
    wv = rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)
    kb = random_words(rng, (B * Hkv, n, 128, 1))
    vb = random_words(rng, (B * Hkv, n, 128, 1))
    ks = (0.3 + rng.random((B * Hkv, n))).astype(np.float16)
    vs = (0.3 + rng.random((B * Hkv, n))).astype(np.float16)
    idx = np.array([[0, 3], [4, 1], [2, 2 + 1], [1, 0]], np.int32)
    out = O.decode_attention(q, wk, wv, kb, vb, ks, vs, idx, tf, win_len=33)
    for b in range(B):
        for h in range(Hkv):
            s = b * Hkv + h
            kr = O.dequantize_original(kb[s][idx[s]], ks[s][idx[s]], tf).reshape(-1, 128)
            vr = O.dequantize_original(vb[s][idx[s]], vs[s][idx[s]], tf).reshape(-1, 128)
            K = torch.from_numpy(np.concatenate([wk[b, h, :33], kr]))
            V = torch.from_numpy(np.concatenate([wv[b, h, :33], vr]))
            g = Hq // Hkv
            Q = torch.from_numpy(q[b, h * g:(h + 1) * g].astype(np.float64))
            ref = torch.nn.functional.scaled_dot_product_attention(Q[None], K[None], V[None])[0]
            assert np.abs(out[b, h * g:(h + 1) * g] - ref.numpy()).max() < 1e-10


def test_dequantize_hand_kat():
    w = np.zeros((1, 128, 1), np.uint64)
    w[0, 0, 0] = np.uint64(0b101)               # channel 0: tokens 0 and 2 are +1
    d = O.dequantize(w, np.float16(0.5))
    assert d.shape == (1, 64, 128)
    assert d[0, 0, 0] == 0.5 and d[0, 1, 0] == -0.5 and d[0, 2, 0] == 0.5 and d[0, 0, 1] == -0.5


def test_bf16_round_kats():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38], np.float32)
    r = O.bf16_round(x)
    assert list(r[:4]) == [1.0, 1.0, 1.0 + 2 ** -6, -2.5]       # ties to even
    assert np.array_equal(r, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_all_small_configs_roundtrip_pipeline(rng):
    """Encode -> score -> top-k -> attention on a tiny store is self-consistent: the tile whose
    keys were set to the query direction ranks first."""
    T, n_tok = 64, 8 * 64
    x = kv_like(rng, (1, n_tok, 128), outliers=False)
    q = rng.standard_normal((1, 4, 128)).astype(np.float32)
    qhat = O.gqa_mean(q, 1)[0]
    x[0, 5 * 64:6 * 64] = 0.8 * qhat / np.linalg.norm(qhat) * 11.3 + 0.2 * x[0, 5 * 64:6 * 64]
    bits, s = O.encode(x, T, O.HADAMARD)
    qbar, _ = O.query_prep(q, 1, O.HADAMARD)
    sc = O.score_tiles(qbar.reshape(-1, 128), bits)
    assert O.topk_tiles(sc, 1)[0, 0] == 5
