"""The tile-store file format (include/kvr_store.h, modules/kvr_store.py) without a GPU: the
library's host-only header codec, section layout and CRC-32, the committed golden store,
corruption handling, and save -> load round trips of TileKVCache / RetrievalIndex state
held in CPU tensors (the same code moves device tensors on the GPU)."""
import io
import struct
import zlib

import numpy as np
import pytest
import torch

from conftest import kv_like
from oracle import kvr_oracle as O


@pytest.fixture(scope="module")
def S():
    from modules import kvr_store
    return kvr_store


@pytest.fixture(scope="module")
def G():
    from tests.golden import make_store_golden as g
    return g


def test_crc32_known_answer_and_zlib(S, rng):
    # the CRC-32 check value of the published catalogue ("123456789" -> 0xCBF43926)
    assert S.crc32(b"123456789") == 0xCBF43926
    assert S.crc32(b"") == 0
    data = rng.integers(0, 256, 10007, dtype=np.uint8).tobytes()
    assert S.crc32(data) == zlib.crc32(data)
    # continuation: crc(a + b) == crc(b, crc(a))
    assert S.crc32(data[5000:], S.crc32(data[:5000])) == zlib.crc32(data)


def _aligned(n):
    return (n + 63) // 64 * 64


@pytest.mark.parametrize("T,win_dtype,counts", [(64, 0, True), (128, 2, False), (64, None, True)])
def test_layout_follows_the_documented_rule(S, T, win_dtype, counts):
    """Section offsets: header 256 bytes, then per layer the present sections in order, each
    starting at a multiple of 64 (restated here from the header's text)."""
    B, Hkv, nt, W, wl, L = 3, 2, 5, 2 * T, 2 * T + 7, 3
    win = win_dtype is not None
    d = S.new_desc(T=T, transform=0, n_layers=L, B=B, Hkv=Hkv, n_tiles=nt, W=W, win_len=wl if win else 0,
                   win_dtype=win_dtype, counts=counts)
    esz = {0: 2, 1: 2, 2: 4}
    sizes = [B * Hkv * nt * 128 * (T // 64) * 8] * 2 + [B * Hkv * nt * 2] * 2 + \
            [B * Hkv * nt * 128 if counts else None] + [B * Hkv * wl * 128 * esz[win_dtype] if win else None] * 2
    off = 256
    for li in range(L):
        for sec, sz in enumerate(sizes):
            if sz is None:
                with pytest.raises(ValueError, match="not in this store"):
                    S.section(d, li, sec)
                continue
            assert S.section(d, li, sec) == (off, sz), (li, sec)
            off = _aligned(off + sz)
    assert S.payload_bytes(d) == off - 256


def test_header_bytes_at_documented_offsets(S):
    d = S.new_desc(T=128, transform=1, n_layers=28, B=4, Hkv=4, n_tiles=1008, W=2048, win_len=2100, win_dtype=0,
                   counts=True, user=(131172, 99, -1, 5))
    d.payload_crc32 = 0xDEADBEEF
    h = S.encode_header(d)
    assert len(h) == 256 and h[:8] == b"KVRSTORE"
    u32 = lambda o: struct.unpack_from("<I", h, o)[0]  # noqa: E731
    i32 = lambda o: struct.unpack_from("<i", h, o)[0]  # noqa: E731
    i64 = lambda o: struct.unpack_from("<q", h, o)[0]  # noqa: E731
    assert (u32(8), u32(12), u32(16)) == (1, 256, 4)
    assert (i32(20), i32(24), i32(28), i32(32), i32(36), i32(40), u32(44), i32(48), u32(52)) == \
           (128, 128, 1, 0, 1, 0, 3, 28, 64)
    assert (i64(56), i64(64), i64(72), i64(80), i64(88)) == (4, 4, 1008, 2048, 2100)
    assert struct.unpack_from("<Q", h, 96)[0] == S.payload_bytes(d)
    assert (u32(104), u32(108)) == (0xDEADBEEF, 0)
    assert [i64(112 + 8 * i) for i in range(4)] == [131172, 99, -1, 5]
    assert h[144:252] == bytes(108)
    assert u32(252) == zlib.crc32(h[:252])
    back = S.decode_header(h)
    for f, _ in S.StoreDesc._fields_:
        if f != "user":
            assert getattr(back, f) == getattr(d, f) or f in ("format_version", "abi_version", "payload_bytes"), f
    assert list(back.user) == [131172, 99, -1, 5]


@pytest.mark.parametrize("field,value,match", [
    ("d", 64, "d=64"), ("T", 32, "T=32"), ("transform", 7, "transform"), ("bit_order", 1, "bit order"),
    ("scale_dtype", 0, "scale dtype"), ("flags", 4, "flags"), ("n_layers", 0, "n_layers"),
    ("Hkv", 0, "sizes"), ("n_tiles", -1, "sizes"), ("W", 65, "multiple"), ("win_len", 192, "win_len"),
    ("win_dtype", 9, "window dtype"), ("B", 1 << 50, "overflow")])
def test_invalid_descriptions_are_rejected(S, field, value, match):
    d = S.new_desc(T=64, transform=0, n_layers=2, B=1, Hkv=2, n_tiles=3, W=128, win_len=130, win_dtype=0)
    setattr(d, field, value)
    with pytest.raises(ValueError, match=match):
        S.encode_header(d)


def test_corrupted_headers_are_rejected(S):
    d = S.new_desc(T=64, transform=0, n_layers=1, B=1, Hkv=2, n_tiles=3, W=64, win_len=64, win_dtype=0)
    h = bytearray(S.encode_header(d))
    for pos in (20, 72, 100, 130, 252):  # any flipped bit fails the header CRC
        bad = bytearray(h)
        bad[pos] ^= 0x10
        with pytest.raises(ValueError, match="CRC"):
            S.decode_header(bytes(bad))
    with pytest.raises(ValueError, match="magic"):
        S.decode_header(b"KVRSTORX" + bytes(h[8:]))
    with pytest.raises(ValueError, match="header bytes"):
        S.decode_header(bytes(h[:200]))
    newer = bytearray(h)
    newer[8:12] = struct.pack("<I", 2)
    newer[252:256] = struct.pack("<I", zlib.crc32(bytes(newer[:252])))
    with pytest.raises(ValueError, match="format version 2"):
        S.decode_header(bytes(newer))
    wrong_size = bytearray(h)
    wrong_size[96:104] = struct.pack("<Q", S.payload_bytes(d) + 64)
    wrong_size[252:256] = struct.pack("<I", zlib.crc32(bytes(wrong_size[:252])))
    with pytest.raises(ValueError, match="payload bytes"):
        S.decode_header(bytes(wrong_size))


def test_golden_store_file(S, G):
    """The committed golden file: the reader returns the oracle's encoding of the seeded
    input, and the writer reproduces the file byte for byte."""
    raw = open(G.PATH, "rb").read()
    desc, layers = S.read_layers(io.BytesIO(raw))
    assert (desc.n_layers, desc.B, desc.Hkv, desc.T, desc.n_tiles, desc.W, desc.win_len) == (1, 1, 1, 64, 2, 64, 66)
    assert list(desc.user) == list(G.USER)
    want = G.golden_sections()
    assert set(layers[0]) == set(want)
    for sec, arr in want.items():
        assert np.array_equal(layers[0][sec].view(np.uint8), np.ascontiguousarray(arr).view(np.uint8)), sec
    buf = io.BytesIO()
    S.write_layers(buf, G.golden_desc(), [want])
    assert buf.getvalue() == raw


def test_truncated_and_corrupted_payload(S, G):
    raw = open(G.PATH, "rb").read()
    with pytest.raises(ValueError, match="truncated"):
        S.read_layers(io.BytesIO(raw[:-10]))
    bad = bytearray(raw)
    bad[256 + 100] ^= 1  # one bit of the K bits
    with pytest.raises(ValueError, match="payload CRC"):
        S.read_layers(io.BytesIO(bytes(bad)))


def _cpu_cache(T, tf, rng, B=2, Hkv=2, W=128, n_prompt=None, dtype=torch.bfloat16):
    """A TileKVCache in CPU tensors filled with the oracle's encoding (ring not at slot 0)."""
    from modules.kvr_cache import TileKVCache
    n_prompt = n_prompt or 3 * T + W + T // 2
    c = TileKVCache(B, Hkv, W, T, tf, "cpu", dtype, tile_cap=8)
    k = O.bf16_round(kv_like(rng, (B * Hkv, n_prompt, 128)))
    v = O.bf16_round(kv_like(rng, (B * Hkv, n_prompt, 128), outliers=False))
    nr = (n_prompt - W) // T * T
    m = nr // T
    kb, ks = O.encode(k[:, :nr], T, tf)
    vb, vs = O.encode(v[:, :nr], T, tf)
    c.kbits[:, :m] = torch.from_numpy(kb.view(np.int64))
    c.vbits[:, :m] = torch.from_numpy(vb.view(np.int64))
    c.kscale[:, :m] = torch.from_numpy(ks)
    c.vscale[:, :m] = torch.from_numpy(vs)
    c.kcount[:, :m] = torch.from_numpy(
        np.unpackbits(kb.view(np.uint8), axis=-1).reshape(kb.shape + (64,)).sum(axis=(-1, -2)).astype(np.uint8))
    r = n_prompt - nr
    start = T  # a ring whose oldest token is not in slot 0
    slots = (np.arange(r) + start) % c.cap
    wk = torch.from_numpy(k[:, nr:].reshape(B, Hkv, r, 128)).to(dtype)
    wv = torch.from_numpy(v[:, nr:].reshape(B, Hkv, r, 128)).to(dtype)
    c.win_k[:, :, slots] = wk
    c.win_v[:, :, slots] = wv
    c.n, c.start, c.n_tiles = r, start, m
    c._push_state()
    return c, wk, wv


@pytest.mark.parametrize("T,tf,dtype", [(64, 0, torch.bfloat16), (128, 1, torch.float32), (64, 0, torch.float16)])
def test_cache_round_trip_cpu(S, rng, T, tf, dtype):
    c, wk, wv = _cpu_cache(T, tf, rng, dtype=dtype)
    raw = S.to_bytes([c, c], user=(5, 6, 7, 8))
    caches, desc = S.from_bytes(raw, "cpu", reserve_tiles=4)
    assert len(caches) == 2 and list(desc.user) == [5, 6, 7, 8]
    for d in caches:
        assert (d.n, d.start, d.n_tiles, d.tile_cap, d.dtype) == (c.n, 0, c.n_tiles, c.n_tiles + 4, dtype)
        m = c.n_tiles
        for name in ("kbits", "vbits", "kscale", "vscale", "kcount"):
            assert torch.equal(getattr(d, name)[:, :m], getattr(c, name)[:, :m]), name
        dk, dv = d.window_tokens()
        assert torch.equal(dk, wk) and torch.equal(dv, wv)
        assert d.state[:, :3].tolist() == [[c.n, 0, c.n_tiles]] * (c.B * c.Hkv)
    # the loaded state decodes as the original (oracle pipeline on both)
    g = np.random.default_rng(3)
    q = O.bf16_round(g.standard_normal((c.B, 8, 128)).astype(np.float32))

    def attend(cc):
        kb = cc.kbits[:, :cc.n_tiles].numpy().view(np.uint64)
        vb = cc.vbits[:, :cc.n_tiles].numpy().view(np.uint64)
        qbar, _ = O.query_prep(q, cc.Hkv, tf)
        idx = O.topk_tiles(O.score_tiles(qbar.reshape(-1, 128), kb), 2)
        wk_, wv_ = cc.window_tokens()
        return O.decode_attention(q, wk_.float().numpy(), wv_.float().numpy(), kb, vb, cc.kscale[:, :cc.n_tiles].numpy(),
                                  cc.vscale[:, :cc.n_tiles].numpy(), idx, tf)
    assert np.array_equal(attend(c), attend(caches[0]))


def test_cache_store_without_counts_rebuilds_them(S, rng):
    c, _, _ = _cpu_cache(64, 0, rng)
    d = S.describe([c])
    d.flags = S.HAS_WINDOW
    wk, wv = c.window_tokens()
    nt = c.n_tiles
    layer = {S.SEC_KBITS: c.kbits[:, :nt], S.SEC_VBITS: c.vbits[:, :nt], S.SEC_KSCALE: c.kscale[:, :nt],
             S.SEC_VSCALE: c.vscale[:, :nt], S.SEC_WIN_K: wk, S.SEC_WIN_V: wv}
    buf = io.BytesIO()
    S.write_layers(buf, d, [layer])
    buf.seek(0)
    (e,), _ = S.load(buf, "cpu")
    assert torch.equal(e.kcount[:, :nt], c.kcount[:, :nt])


def test_mismatched_layers_and_sections_are_rejected(S, rng):
    c, _, _ = _cpu_cache(64, 0, rng)
    c2, _, _ = _cpu_cache(64, 0, rng, n_prompt=3 * 64 + 128 + 40)
    with pytest.raises(ValueError, match="same shape and state"):
        S.to_bytes([c, c2])
    d = S.describe([c])
    with pytest.raises(ValueError, match="bytes, the layout needs"):
        S.write_layers(io.BytesIO(), d, [{sec: np.zeros(3, np.uint8) for sec in S.SECTIONS}])


def test_retrieval_index_round_trip_cpu(S, rng):
    from modules.kvr_retrieval import RetrievalIndex
    ri = RetrievalIndex(2, 128, device="cpu", tile=64)
    ri._calibrated = True
    k = O.bf16_round(kv_like(rng, (2, 192, 128)))
    kb, ks = O.encode(k, 64, O.HADAMARD)
    vb, vs = O.encode(k[::-1].copy(), 64, O.HADAMARD)
    ri.kbits[:, :3] = torch.from_numpy(kb.view(np.int64))
    ri.vbits[:, :3] = torch.from_numpy(vb.view(np.int64))
    ri.kscale[:, :3] = torch.from_numpy(ks)
    ri.vscale[:, :3] = torch.from_numpy(vs)
    ri.n_tiles = 3
    ri.tail_k = torch.from_numpy(kv_like(rng, (17, 2, 128)))
    ri.tail_v = torch.from_numpy(kv_like(rng, (17, 2, 128)))
    buf = io.BytesIO()
    desc = ri.save_store(buf)
    assert (desc.W, desc.win_len, desc.flags, desc.win_dtype) == (0, 17, S.HAS_WINDOW, 2)
    buf.seek(0)
    r2 = RetrievalIndex(2, 128, device="cpu", tile=64)
    r2.load_store(buf)
    assert r2.n_tiles == 3 and r2.n_stored == ri.n_stored and r2._calibrated
    for name in ("kbits", "vbits", "kscale", "vscale"):
        assert torch.equal(getattr(r2, name)[:, :3], getattr(ri, name)[:, :3]), name
    assert torch.equal(r2.tail_k, ri.tail_k) and torch.equal(r2.tail_v, ri.tail_v)
    buf.seek(0)
    with pytest.raises(ValueError, match="does not match"):
        RetrievalIndex(4, 128, device="cpu", tile=64).load_store(buf)
    buf.seek(0)
    with pytest.raises(ValueError, match="no cache window"):
        S.load(buf, "cpu")
