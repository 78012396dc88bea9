"""GPU parity of the cache-side paths: the fp32 window, the ring window, the live (device-
resident) state of the decode step, the fused ring append (kvr_cache_append), the bounded
waits' failure reporting, and candidate-list tags across workspace layout changes.

Bars as in test_gpu_parity: bits and scales bit-exact, top-k index-exact (Hadamard), attention
within 1e-5 max-abs (fp32 out) / 2e-3 + 2^-8 |ref| (bf16 out) of the float64 oracle; paths that
must run the same kernels on the same data (live state vs host arguments, append vs encode)
are compared bit for bit.
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


def check_out(out, ref, what):
    o = out.float().cpu().numpy()
    if out.dtype == torch.float32:
        err = np.abs(o - ref).max()
        assert err <= 1e-5, f"{what}: fp32 max-abs {err}"
    else:
        excess = (np.abs(o - ref) - (2e-3 + np.abs(ref) * 2.0 ** -8)).max()
        assert excess <= 0, f"{what}: bf16 error exceeds 2e-3 + 2^-8|ref| by {excess}"


def make_layer(H, rng, B, Hkv, n_tiles, T, tf, counts=True):
    n_tok = n_tiles * T
    K = torch.from_numpy(kv_like(rng, (B, Hkv, n_tok, 128))).to(DEV, torch.bfloat16)
    V = torch.from_numpy(rng.standard_normal((B, Hkv, n_tok, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    kc = H.alloc_counts(B * Hkv, n_tiles, DEV) if counts else None
    kb, ks = H.encode_tiles(K, T, tf, counts=kc)
    vb, vs = H.encode_tiles(V, T, tf)
    return kb, vb, ks, vs, kc


# ----------------------------------------------------------------------------- fp32 window

@pytest.mark.parametrize("T,tf", [(64, O.HADAMARD), (128, O.DCT)])
@pytest.mark.parametrize("qdt", ["fp32", "bf16"])
def test_fp32_window_decode_step(H, rng, T, tf, qdt):
    """An fp32 window (fp32 MFMA) inside the full decode step, against the float64 oracle."""
    say(f"[fp32 window] T={T} tf={tf} q={qdt}")
    B, Hq, Hkv, W, n_tiles, k = 2, 32, 8, 300, 12, 4
    kb, vb, ks, vs, kc = make_layer(H, rng, B, Hkv, n_tiles, T, tf)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, TDT[qdt])
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, W, 128))).to(DEV)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV)
    idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
    out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, tf, k, out_dtype=torch.float32, idx_out=idx,
                        kcounts=kc)
    torch.cuda.synchronize()
    qn = q.float().cpu().numpy()
    ig = idx.cpu().numpy()
    if tf == O.HADAMARD:
        qbar, _ = O.query_prep(qn, Hkv, tf)
        assert np.array_equal(ig, O.topk_tiles(O.score_tiles(qbar.reshape(-1, 128), u64(kb)), k))
    ref = O.decode_attention(qn, wk.cpu().numpy(), wv.cpu().numpy(), u64(kb), u64(vb), ks.cpu().numpy(),
                             vs.cpu().numpy(), ig, tf)
    check_out(out, ref, "fp32 window step")
    # window only, through the launch chain (kvr_decode_attn), against torch's SDPA in fp32
    out_w = H.decode_attn(q, wk, wv, W, None, None, None, None, None, T, tf, out_dtype=torch.float32)
    sdpa = torch.nn.functional.scaled_dot_product_attention(q.float().view(B, Hkv, Hq // Hkv, 128), wk, wv)
    assert (out_w.view(B, Hkv, Hq // Hkv, 128) - sdpa).abs().max().item() < 1e-5


# ----------------------------------------------------------------------------- ring window

@pytest.mark.parametrize("wdt", ["bf16", "fp32"])
def test_ring_window_equals_unrolled(H, rng, wdt):
    """A ring window (tokens from slot win_start, wrapping) attends exactly like the same
    tokens laid out in order."""
    say(f"[ring] {wdt}")
    B, Hq, Hkv, T, n_tiles, k = 2, 32, 8, 64, 9, 3
    cap, n, start = 320, 290, 256
    kb, vb, ks, vs, kc = make_layer(H, rng, B, Hkv, n_tiles, T, O.HADAMARD)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    ring_k = torch.from_numpy(kv_like(rng, (B, Hkv, cap, 128))).to(DEV, TDT[wdt])
    ring_v = torch.from_numpy(rng.standard_normal((B, Hkv, cap, 128)).astype(np.float32)).to(DEV, TDT[wdt])
    order = (torch.arange(n, device=DEV) + start) % cap
    flat_k, flat_v = ring_k[:, :, order].contiguous(), ring_v[:, :, order].contiguous()
    outs = []
    for wk, wv, w0, wc in ((ring_k, ring_v, start, cap), (flat_k, flat_v, 0, 0)):
        idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
        outs.append((H.decode_step(q, wk, wv, n, kb, vb, ks, vs, n_tiles, T, H.HADAMARD, k, out_dtype=torch.float32,
                                   idx_out=idx, kcounts=kc, win_start=w0, win_cap=wc), idx))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][1], outs[1][1])
    ref = O.decode_attention(q.float().cpu().numpy(), flat_k.float().cpu().numpy(), flat_v.float().cpu().numpy(),
                             u64(kb), u64(vb), ks.cpu().numpy(), vs.cpu().numpy(), outs[0][1].cpu().numpy(),
                             O.HADAMARD)
    check_out(outs[0][0], ref, "ring")
    check_out(outs[1][0], ref, "unrolled")


# ----------------------------------------------------------------------------- live state

@pytest.mark.parametrize("T,tf", [(64, O.HADAMARD), (128, O.DCT)])
def test_live_state_equals_host_arguments(H, rng, T, tf):
    """Reading the window length, ring start and tile count from the device state runs the
    same work as passing them from the host (with the ring's tokens laid out in order, the
    one-launch step's plain-window form): identical tiles selected and identical outputs,
    for live counts below the capacities the launch is sized for (and fewer live tiles
    than k: every stored tile is taken).  A ring without a live state (the launch chain)
    selects the same tiles and meets the oracle's bar."""
    say(f"[live] T={T} tf={tf}")
    B, Hq, Hkv, k = 2, 28 if tf == O.DCT else 32, 4 if tf == O.DCT else 8, 5
    W = 2 * T
    cap, tile_cap = W + T, 20
    kb, vb, ks, vs, kc = make_layer(H, rng, B, Hkv, tile_cap, T, tf)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    ring_k = torch.from_numpy(kv_like(rng, (B, Hkv, cap, 128))).to(DEV, torch.bfloat16)
    ring_v = torch.from_numpy(rng.standard_normal((B, Hkv, cap, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    ws = H.decode_step_workspace(B, Hq, Hkv, cap - 1, tile_cap, k, T, DEV)
    for n, start, n_tiles in [(W, 0, 20), (W + T - 1, T, 17), (W + 5, 2 * T, 3), (W, T, 1)]:
        state = torch.tensor([[n, start, n_tiles, 0]] * (B * Hkv), dtype=torch.int32, device=DEV)
        idx_l = torch.full((B * Hkv, k), -7, dtype=torch.int32, device=DEV)
        out_l = H.decode_step(q, ring_k, ring_v, cap - 1, kb, vb, ks, vs, tile_cap, T, tf, k, out_dtype=torch.float32,
                              idx_out=idx_l, workspace=ws, kcounts=kc, win_cap=cap, live_state=state)
        ke = min(k, n_tiles)
        order = (torch.arange(n, device=DEV) + start) % cap
        flat_k, flat_v = ring_k[:, :, order].contiguous(), ring_v[:, :, order].contiguous()
        idx_h = torch.empty((B * Hkv, ke), dtype=torch.int32, device=DEV)
        out_h = H.decode_step(q, flat_k, flat_v, n, kb, vb, ks, vs, n_tiles, T, tf, ke, out_dtype=torch.float32,
                              idx_out=idx_h, kcounts=kc)
        idx_c = torch.empty((B * Hkv, ke), dtype=torch.int32, device=DEV)
        out_c = H.decode_step(q, ring_k, ring_v, n, kb, vb, ks, vs, n_tiles, T, tf, ke, out_dtype=torch.float32,
                              idx_out=idx_c, kcounts=kc, win_start=start, win_cap=cap)
        torch.cuda.synchronize()
        il = idx_l.cpu().numpy()
        assert np.array_equal(il[:, :ke], idx_h.cpu().numpy()), (n, start, n_tiles)
        assert np.array_equal(il[:, :ke], idx_c.cpu().numpy()), (n, start, n_tiles)
        assert (il[:, ke:] == -1).all()
        per = max(8 * 64 // T, 4)  # selected tiles per retrieved item
        if -(-k // per) == -(-ke // per):  # the same partial records: the same sums, bit for bit
            assert torch.equal(out_l, out_h), (n, start, n_tiles)
        # (with more retrieved items than tiles, the live launch merges an extra empty record:
        # the same value up to the order of the merge's sums, held to the oracle's bar below)
        assert H.workspace_status(ws) == 0
        ref = O.decode_attention(q.float().cpu().numpy(), ring_k[:, :, order].float().cpu().numpy(),
                                 ring_v[:, :, order].float().cpu().numpy(), u64(kb), u64(vb), ks.cpu().numpy(),
                                 vs.cpu().numpy(), il[:, :ke], tf)
        check_out(out_l, ref, f"live n={n} start={start} n_tiles={n_tiles}")
        check_out(out_c, ref, f"ring, launch chain n={n} start={start} n_tiles={n_tiles}")


# ----------------------------------------------------------------------------- ring append

@pytest.mark.parametrize("T,tf,wdt", [(64, O.HADAMARD, "bf16"), (128, O.HADAMARD, "fp16"), (64, O.DCT, "bf16"),
                                       (128, O.DCT, "bf16"), (64, O.HADAMARD, "fp32")])
def test_cache_append_matches_encode(H, rng, T, tf, wdt):
    """kvr_cache_append over several evictions: the window ring holds the last tokens in
    order, the state follows the host rule, and the tiles (bits, scales, channel counts) are
    bit-identical to kvr_encode_tiles on the same tokens (Hadamard: and to the oracle)."""
    say(f"[append] T={T} tf={tf} window={wdt}")
    B, Hkv, W = 2, 3, 2 * T
    cap = W + T
    n0, n_app = W + 10, 3 * T + 7
    n_all = n0 + n_app
    x_k = torch.from_numpy(kv_like(rng, (B, Hkv, n_all, 128))).to(DEV, TDT[wdt])
    x_v = torch.from_numpy(rng.standard_normal((B, Hkv, n_all, 128)).astype(np.float32)).to(DEV, TDT[wdt])
    win_k = torch.zeros((B, Hkv, cap, 128), dtype=TDT[wdt], device=DEV)
    win_v = torch.zeros_like(win_k)
    tile_cap = 8
    kb, ks = H.alloc_store(B * Hkv, tile_cap, T, DEV)
    vb, vs = H.alloc_store(B * Hkv, tile_cap, T, DEV)
    kc = H.alloc_counts(B * Hkv, tile_cap, DEV)
    win_k[:, :, :n0] = x_k[:, :, :n0]
    win_v[:, :, :n0] = x_v[:, :, :n0]
    state = torch.tensor([[n0, 0, 0, 0]] * (B * Hkv), dtype=torch.int32, device=DEV)
    n, start, nt = n0, 0, 0
    for t in range(n0, n_all):
        H.cache_append(x_k[:, :, t], x_v[:, :, t], win_k, win_v, W, T, tf, kb, vb, ks, vs, kc, state)
        if n + 1 == cap:
            n, start, nt = W, (start + T) % cap, nt + 1
        else:
            n += 1
    torch.cuda.synchronize()
    st = state.cpu().numpy()
    assert (st == np.array([n, start, nt, 0])).all(), (st[0], (n, start, nt))
    assert nt == 3
    order = (torch.arange(n, device=DEV) + start) % cap
    assert torch.equal(win_k[:, :, order], x_k[:, :, nt * T:n_all])
    assert torch.equal(win_v[:, :, order], x_v[:, :, nt * T:n_all])
    rkc = H.alloc_counts(B * Hkv, nt, DEV)
    rkb, rks = H.encode_tiles(x_k[:, :, :nt * T], T, tf, counts=rkc)
    rvb, rvs = H.encode_tiles(x_v[:, :, :nt * T], T, tf)
    torch.cuda.synchronize()
    assert torch.equal(kb[:, :nt], rkb) and torch.equal(ks[:, :nt], rks) and torch.equal(kc[:, :nt], rkc)
    assert torch.equal(vb[:, :nt], rvb) and torch.equal(vs[:, :nt], rvs)
    assert not kb[:, nt:].any()
    if tf == O.HADAMARD:
        rb, rs = O.encode(x_k[:, :, :nt * T].float().cpu().numpy().reshape(B * Hkv, nt * T, 128), T, O.HADAMARD)
        assert np.array_equal(u64(kb[:, :nt]), rb)
        assert np.array_equal(ks[:, :nt].cpu().numpy().view(np.uint16), rs.view(np.uint16))


def test_cache_append_full_store_and_bad_state_are_reported(H, rng):
    say("[append] full store -> error 2, invalid state -> error 1, nothing out of bounds")
    B, Hkv, T, W = 1, 2, 64, 64
    cap = W + T
    win_k = torch.zeros((B, Hkv, cap, 128), dtype=torch.bfloat16, device=DEV)
    win_v = torch.zeros_like(win_k)
    kb, ks = H.alloc_store(B * Hkv, 1, T, DEV)
    vb, vs = H.alloc_store(B * Hkv, 1, T, DEV)
    x = torch.from_numpy(kv_like(rng, (B, Hkv, 128))).to(DEV, torch.bfloat16)
    state = torch.tensor([[cap - 1, 0, 1, 0]] * (B * Hkv), dtype=torch.int32, device=DEV)  # store already full
    H.cache_append(x, x, win_k, win_v, W, T, H.HADAMARD, kb, vb, ks, vs, None, state)
    torch.cuda.synchronize()
    assert (state.cpu().numpy() == np.array([W, T, 1, 2])).all()
    assert not kb.any()
    state = torch.tensor([[cap, 0, 0, 0]] * (B * Hkv), dtype=torch.int32, device=DEV)  # n out of range
    H.cache_append(x, x, win_k, win_v, W, T, H.HADAMARD, kb, vb, ks, vs, None, state)
    torch.cuda.synchronize()
    assert (state.cpu().numpy() == np.array([cap, 0, 0, 1])).all()


# ----------------------------------------------------------------------------- failure reporting

def test_bounded_wait_give_up_is_loud(H, rng):
    """Forced from the host (every wait of the one-launch step expects a tag no list
    carries, 16 polls): every kernel ends normally, the outputs of every segment are NaN,
    the workspace status word is set and check_workspace raises (and re-zeroes the
    workspace); with the default restored the same workspace gives the oracle's answer."""
    say("[give-up] forced bounded-wait failure")
    B, Hq, Hkv, T, n_tiles, k, W = 2, 32, 8, 64, 20, 4, 128
    kb, vb, ks, vs, kc = make_layer(H, rng, B, Hkv, n_tiles, T, O.HADAMARD)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, W, 128))).to(DEV, torch.bfloat16)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    ws = H.decode_step_workspace(B, Hq, Hkv, W, n_tiles, k, T, DEV)
    try:
        H.set_wait_limit(16, force_give_up=True)
        out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, H.HADAMARD, k, out_dtype=torch.float32,
                            workspace=ws, kcounts=kc)
        torch.cuda.synchronize()
    finally:
        H.set_wait_limit(0, force_give_up=False)
    assert torch.isnan(out).all()
    assert H.workspace_status(ws) == 1
    with pytest.raises(RuntimeError, match="gave up"):
        H.check_workspace(ws)
    assert H.workspace_status(ws) == 0
    idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
    out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, H.HADAMARD, k, out_dtype=torch.float32,
                        workspace=ws, kcounts=kc, idx_out=idx)
    torch.cuda.synchronize()
    assert H.workspace_status(ws) == 0
    ref = O.decode_attention(q.float().cpu().numpy(), wk.float().cpu().numpy(), wv.float().cpu().numpy(),
                             u64(kb), u64(vb), ks.cpu().numpy(), vs.cpu().numpy(), idx.cpu().numpy(), O.HADAMARD)
    check_out(out, ref, "after recovery")


def test_tile_cache_reports_give_up(H, rng):
    """The product path raises: TileKVCache.check() after a forced give-up."""
    import modules
    say("[give-up] TileKVCache.check raises")
    B, Hkv, Hq, W, T = 1, 2, 8, 64, 64
    c = modules.TileKVCache(B, Hkv, W, T, H.HADAMARD, DEV, torch.bfloat16, tile_cap=4)
    x = torch.from_numpy(kv_like(rng, (B, Hkv, 3 * T, 128))).to(DEV, torch.bfloat16)
    c.load_prompt(x, x)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    try:
        H.set_wait_limit(8, force_give_up=True)
        out = c.attend(q, 128)
        torch.cuda.synchronize()
    finally:
        H.set_wait_limit(0, force_give_up=False)
    assert torch.isnan(out.float()).all()
    with pytest.raises(RuntimeError, match="gave up"):
        c.check()
    out = c.attend(q, 128)
    c.check()
    assert torch.isfinite(out.float()).all()


# ----------------------------------------------------------------------------- tags across layouts

def test_candidate_tags_across_growing_layouts(H, rng):
    """One workspace, the tile count growing every call (as a cache's store grows, which
    shifts the score and candidate regions inside the reused workspace) and shrinking back:
    no bounded wait gives up and every call matches the oracle's selection and output."""
    say("[tags] growing n_tiles on one workspace")
    B, Hq, Hkv, T, k, W = 2, 32, 8, 64, 8, 192
    n_max = 300
    kb, vb, ks, vs, kc = make_layer(H, rng, B, Hkv, n_max, T, O.HADAMARD)
    wk = torch.from_numpy(kv_like(rng, (B, Hkv, W, 128))).to(DEV, torch.bfloat16)
    wv = torch.from_numpy(rng.standard_normal((B, Hkv, W, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
    ws = H.decode_step_workspace(B, Hq, Hkv, W, n_max, k, T, DEV)
    kbn, vbn, ksn, vsn = u64(kb), u64(vb), ks.cpu().numpy(), vs.cpu().numpy()
    for it, n_tiles in enumerate([10, 64, 128, 129, 200, 255, 256, 257, 300, 120, 300]):
        q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)
        idx = torch.empty((B * Hkv, k), dtype=torch.int32, device=DEV)
        out = H.decode_step(q, wk, wv, W, kb, vb, ks, vs, n_tiles, T, H.HADAMARD, k, out_dtype=torch.float32,
                            idx_out=idx, workspace=ws, kcounts=kc)
        torch.cuda.synchronize()
        assert H.workspace_status(ws) == 0, n_tiles
        qn = q.float().cpu().numpy()
        qbar, _ = O.query_prep(qn, Hkv, O.HADAMARD)
        iref = O.topk_tiles(O.score_tiles(qbar.reshape(-1, 128), kbn[:, :n_tiles]), k)
        assert np.array_equal(idx.cpu().numpy(), iref), n_tiles
        ref = O.decode_attention(qn, wk.float().cpu().numpy(), wv.float().cpu().numpy(), kbn[:, :n_tiles],
                                 vbn[:, :n_tiles], ksn[:, :n_tiles], vsn[:, :n_tiles], iref, O.HADAMARD)
        check_out(out, ref, f"n_tiles={n_tiles}")
