"""Golden fixtures (tests/golden/golden_*.npz, written by tests/golden/make_golden.py): the CPU
oracle still reproduces them, and the HIP path (through the C ABI) matches them -- codec
bits/scales (Hadamard bit-exact; DCT, whose rotation is a tolerance, up to rare sign flips
near zero), tile scores bit-exact given the stored rotated query, top-k indices exact,
attention within 1e-5 (fp32 output), and the one-launch decode step end to end."""
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402

from oracle import kvr_oracle as O  # noqa: E402

NAMES = sorted(G.CASES)


def load(name):
    return dict(np.load(os.path.join(HERE, "golden", f"golden_{name}.npz")))


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    T, tf, seed = G.CASES[name]
    g = load(name)
    K, V, q, win_k, win_v = G.inputs(T, seed)
    assert np.uint64(g["input_checksum"]) == G.checksum(K, V, q, win_k, win_v), "input generator drifted"
    r = G.outputs(T, tf, seed)
    for key in ("kbits", "kscale", "vbits", "vscale", "qbar", "scores", "idx"):
        assert np.array_equal(np.asarray(r[key]).view(np.uint8), g[key].view(np.uint8)), key
    assert np.abs(r["out"] - g["out"]).max() < 1e-12


# ----------------------------------------------------------------------------- GPU

DEV = "cuda"


@pytest.fixture(scope="module")
def H():
    from modules import _hip
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    _hip.lib()
    return _hip


def bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV, torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_encode_matches_golden(H, name):
    T, tf, seed = G.CASES[name]
    g = load(name)
    K, V, _, _, _ = G.inputs(T, seed)
    for x, kb, ks in ((K, "kbits", "kscale"), (V, "vbits", "vscale")):
        bits, scales = H.encode_tiles(bf16(x)[None], T, tf)
        torch.cuda.synchronize()
        b = bits.cpu().numpy().view(np.uint64)
        s = scales.cpu().numpy()
        if tf == O.HADAMARD:
            assert np.array_equal(b, g[kb]) and np.array_equal(s.view(np.uint16), g[ks].view(np.uint16))
        else:  # fp32 rotation order differs from the float64 oracle: rare flips of |y| ~ 0
            flips = np.unpackbits((b ^ g[kb]).view(np.uint8)).sum()
            assert flips <= 1e-3 * b.size * 64, flips
            assert np.allclose(s.astype(np.float32), g[ks].astype(np.float32), rtol=2e-3, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_scores_topk_attention_match_golden(H, name):
    T, tf, seed = G.CASES[name]
    g = load(name)
    _, _, q, win_k, win_v = G.inputs(T, seed)
    kbits = torch.from_numpy(g["kbits"].view(np.int64)).to(DEV)
    vbits = torch.from_numpy(g["vbits"].view(np.int64)).to(DEV)
    kscale = torch.from_numpy(g["kscale"]).to(DEV)
    vscale = torch.from_numpy(g["vscale"]).to(DEV)
    qbar = torch.from_numpy(g["qbar"]).to(DEV)
    n_tiles = g["kbits"].shape[1]
    scores = H.score_tiles(qbar, kbits, n_tiles, T)
    idx = H.topk_tiles(scores, g["idx"].shape[1])
    torch.cuda.synchronize()
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), g["scores"].view(np.uint32))
    assert np.array_equal(idx.cpu().numpy(), g["idx"])
    out = H.decode_attn(bf16(q), bf16(win_k), bf16(win_v), win_k.shape[2], kbits, vbits, kscale, vscale,
                        torch.from_numpy(g["idx"]).to(DEV), T, tf, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - g["out"]).max() < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_decode_step_matches_golden(H, name):
    T, tf, seed = G.CASES[name]
    g = load(name)
    _, _, q, win_k, win_v = G.inputs(T, seed)
    kbits = torch.from_numpy(g["kbits"].view(np.int64)).to(DEV)
    vbits = torch.from_numpy(g["vbits"].view(np.int64)).to(DEV)
    kscale = torch.from_numpy(g["kscale"]).to(DEV)
    vscale = torch.from_numpy(g["vscale"]).to(DEV)
    k = g["idx"].shape[1]
    idx = torch.empty((g["idx"].shape[0], k), dtype=torch.int32, device=DEV)
    out = H.decode_step(bf16(q), bf16(win_k), bf16(win_v), win_k.shape[2], kbits, vbits, kscale, vscale,
                        g["kbits"].shape[1], T, tf, k, out_dtype=torch.float32, idx_out=idx)
    torch.cuda.synchronize()
    assert np.array_equal(np.sort(idx.cpu().numpy(), axis=1), np.sort(g["idx"], axis=1))
    assert np.abs(out.cpu().numpy() - g["out"]).max() < 1e-5
