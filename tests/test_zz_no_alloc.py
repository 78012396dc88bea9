"""The allocation-free decode step (kvr_decode_step_noalloc, scratch in the library's per-GPU
device array) against the workspace entry point kvr_decode_step, through the C ABI.

Both run the same kernels on the same inputs, so the selected tiles and the outputs must be
identical bit for bit; each call is also held to the oracle's bar (index-exact top-k,
attention within 1e-5 fp32 / 2e-3 + 2^-8 |ref| bf16).  Calls follow one another on one GPU
with shrinking sizes (the scratch keeps the last call's contents), and a live-state call
(graph-capturable form) is included.  Sizes beyond the scratch are rejected before any
launch.
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


def gen(shape, seed, outliers=True):
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


CASES = [  # B, Hq, Hkv, n_tiles, W, T, k, transform, out dtype -- sizes shrink call by call
    (8, 32, 8, 240, 1024, 64, 32, O.HADAMARD, torch.bfloat16),
    (2, 32, 8, 60, 256, 64, 8, O.HADAMARD, torch.float32),
    (1, 28, 4, 40, 256, 128, 16, O.DCT, torch.float32),
]


def test_noalloc_equals_workspace_entry_point(H):
    for i, (B, Hq, Hkv, n_tiles, W, T, k, tf, odt) in enumerate(CASES):
        say(f"[noalloc] call {i}: B={B} Hq={Hq} Hkv={Hkv} n_tiles={n_tiles} W={W} T={T} k={k} tf={tf} out={odt}")
        need = H.lib().kvr_decode_step_workspace(B, Hq, Hkv, W, n_tiles, k, T)
        assert 0 < need <= H.NOALLOC_SCRATCH_BYTES
        K = gen((B, Hkv, n_tiles * T, 128), 100 + i)
        V = gen((B, Hkv, n_tiles * T, 128), 200 + i, outliers=False)
        kc = H.alloc_counts(B * Hkv, n_tiles, DEV)
        kb, ks = H.encode_tiles(K, T, tf, counts=kc)
        vb, vs = H.encode_tiles(V, T, tf)
        wk = gen((B, Hkv, W, 128), 300 + i)
        wv = gen((B, Hkv, W, 128), 400 + i, outliers=False)
        q = gen((B, Hq, 128), 500 + i, outliers=False)
        idx_w = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
        idx_n = torch.full((B * Hkv, k), -9, dtype=torch.int32, device=DEV)
        out_w = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=odt, idx_out=idx_w,
                              kcounts=kc)
        out_n = H.decode_step_noalloc(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=odt, idx_out=idx_n,
                                      kcounts=kc)
        torch.cuda.synchronize()
        assert torch.equal(idx_n, idx_w), i
        assert torch.equal(out_n, out_w), i
        qn = q.float().cpu().numpy()
        qbar, _ = O.query_prep(qn, Hkv, tf)
        sref = O.score_tiles(qbar.reshape(-1, 128), u64(kb))
        ig = idx_n.cpu().numpy()
        if tf == O.HADAMARD:
            assert np.array_equal(ig, O.topk_tiles(sref, k))
        ref = O.decode_attention(qn, wk.float().cpu().numpy(), wv.float().cpu().numpy(), u64(kb), u64(vb),
                                 ks.cpu().numpy(), vs.cpu().numpy(), ig, tf)
        check_out(out_n, ref, f"noalloc call {i}")


def test_noalloc_live_state(H):
    """The graph-capturable form: ring window and live device state, twice in a row with
    different live counts, equal to the workspace entry point."""
    say("[noalloc] live state")
    B, Hq, Hkv, T, k = 2, 32, 8, 64, 6
    W = 4 * T
    cap, tile_cap = W + T, 30
    K = gen((B, Hkv, tile_cap * T, 128), 600)
    V = gen((B, Hkv, tile_cap * T, 128), 601, outliers=False)
    kc = H.alloc_counts(B * Hkv, tile_cap, DEV)
    kb, ks = H.encode_tiles(K, T, H.HADAMARD, counts=kc)
    vb, vs = H.encode_tiles(V, T, H.HADAMARD)
    rk = gen((B, Hkv, cap, 128), 602)
    rv = gen((B, Hkv, cap, 128), 603, outliers=False)
    q = gen((B, Hq, 128), 604, outliers=False)
    for n, start, nt in [(W + T - 1, 2 * T, 30), (W + 3, T, 12)]:
        state = torch.tensor([[n, start, nt, 0]] * (B * Hkv), dtype=torch.int32, device=DEV)
        outs = []
        for fn in (H.decode_step, H.decode_step_noalloc):
            idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
            outs.append((fn(q, rk, rv, cap - 1, kb, vb, ks, vs, tile_cap, T, H.HADAMARD, k, out_dtype=torch.float32,
                            idx_out=idx, kcounts=kc, win_cap=cap, live_state=state), idx))
        torch.cuda.synchronize()
        assert torch.equal(outs[0][1], outs[1][1]) and torch.equal(outs[0][0], outs[1][0]), (n, start, nt)


def test_noalloc_rejects_sizes_beyond_scratch(H):
    say("[noalloc] oversize request rejected before any launch")
    B, Hq, Hkv, W, n_tiles, k, T = 64, 32, 8, 4096, 4000, 64, 64
    assert H.lib().kvr_decode_step_workspace(B, Hq, Hkv, W, n_tiles, k, T) > H.NOALLOC_SCRATCH_BYTES
    q = torch.zeros((B, Hq, 128), dtype=torch.bfloat16, device=DEV)
    wk = torch.zeros((1, Hkv, 8, 128), dtype=torch.bfloat16, device=DEV).expand(B, Hkv, 8, 128)
    kb, ks = H.alloc_store(1, 1, T, DEV)
    with pytest.raises(RuntimeError, match="allocation-free entry point holds"):
        H.lib()  # loaded
        rc = H.lib().kvr_decode_step_noalloc(
            H._ptr(q), H.BF16, B, Hq, Hkv, 128, H._ptr(wk), H._ptr(wk), H.BF16, W, 0, 0, 0, 0, 128, H._ptr(kb),
            H._ptr(kb), H._ptr(ks), H._ptr(ks), None, n_tiles, n_tiles, T, H.HADAMARD, None, None, k, None,
            H._ptr(q), H.BF16, None, H._stream())
        H.check(rc, "kvr_decode_step_noalloc")
    assert rc == -3
