"""Tile-store files on the GPU: a TileKVCache (and a KVRHook's every layer) saved after it was
filled and decoded by the HIP kernels, loaded into new device buffers, decodes bit for bit as
the original -- at once and after further appends that evict tokens into new tiles."""
import io

import numpy as np
import pytest
import torch

from conftest import kv_like

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def M():
    import modules
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    modules._hip.lib()
    return modules


def _tok(rng, B, Hkv, n, outliers=True):
    return torch.from_numpy(kv_like(rng, (B, Hkv, n, 128), outliers)).to(DEV, torch.bfloat16)


@pytest.mark.parametrize("T,tf_name,dtype", [(64, "hadamard", torch.bfloat16), (128, "dct", torch.bfloat16),
                                             (64, "hadamard", torch.float32)])
def test_cache_save_load_decodes_identically(M, rng, T, tf_name, dtype):
    from modules import kvr_store
    from modules.kvr_cache import TileKVCache
    tf = M._hip.TRANSFORMS[tf_name]
    B, Hkv, Hq, W = 2, 2, 8, 256
    say(f"[store] T={T} {tf_name} window {dtype}")
    L = W + 5 * T + 10
    c = TileKVCache(B, Hkv, W, T, tf, DEV, dtype, tile_cap=16)
    c.load_prompt(_tok(rng, B, Hkv, L), _tok(rng, B, Hkv, L, False))
    extra = [(_tok(rng, B, Hkv, 1)[:, :, 0], _tok(rng, B, Hkv, 1, False)[:, :, 0]) for _ in range(3 * T)]
    for kk, vv in extra[:T]:  # the ring start moves off slot 0
        c.append(kk, vv)
    assert c.start != 0
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(DEV, torch.bfloat16)

    def attend(cc):
        idx = torch.empty((B * Hkv, 4), dtype=torch.int32, device=DEV)
        out = cc.attend(q, 4 * T, out_dtype=torch.float32, idx_out=idx)
        return out, idx

    o1, i1 = attend(c)
    raw = kvr_store.to_bytes([c], user=(1, 2, 3, 4))
    (d,), desc = kvr_store.from_bytes(raw, DEV, reserve_tiles=8)
    assert (d.n, d.start, d.n_tiles) == (c.n, 0, c.n_tiles) and list(desc.user) == [1, 2, 3, 4]
    o2, i2 = attend(d)
    torch.cuda.synchronize()
    assert torch.equal(i1, i2)
    assert torch.equal(o1, o2)
    for kk, vv in extra[T:]:  # two more evictions on both
        c.append(kk, vv)
        d.append(kk, vv)
    assert d.n_tiles == c.n_tiles
    o3, i3 = attend(c)
    o4, i4 = attend(d)
    torch.cuda.synchronize()
    m = c.n_tiles
    for name in ("kbits", "vbits", "kscale", "vscale", "kcount"):
        assert torch.equal(getattr(c, name)[:, :m], getattr(d, name)[:, :m]), name
    assert torch.equal(i3, i4) and torch.equal(o3, o4)
    c.check()
    d.check()


def test_hook_state_save_load_continues_identically(M):
    """Prefix caching: a hook's state saved after prefill and loaded into a second hook on the
    same model decodes the same tokens to identical logits, with retrieval active."""
    from test_gpu_api import tiny_llama, token_ids
    say("[store] KVRHook save_state / load_state")
    model = tiny_llama()
    B, L, W, T, steps = 1, 300, 128, 64, 24  # the window (172 of 192 slots) evicts a tile on step 21
    full = token_ids(B, L + steps, seed=31)
    a = M.KVRHook(model, window_size=W, top_k=128, tile=T, num_denoise_steps=0)
    a.prefill(full[:, :L])
    buf = io.BytesIO()
    a.save_state(buf)
    buf.seek(0)
    b = M.KVRHook(model, window_size=W, top_k=128, tile=T, num_denoise_steps=0)
    desc = b.load_state(buf)
    assert desc.n_layers == 2 and b._context_len == L and b.caches[0].n_tiles == 2

    def run(h):
        logits = []
        h.register()
        try:
            for s in range(steps):
                with torch.no_grad():
                    logits.append(model(full[:, L - 1 + s:L + s], use_cache=False).logits[:, -1].float())
                h._step += 1
                h._context_len += 1
        finally:
            h.remove()
        h.check()
        return torch.stack(logits)

    la = run(a)
    lb = run(b)
    assert a.caches[0].n_tiles == 3  # an eviction happened during the steps
    assert torch.equal(la, lb)
