"""Tile-store files: the decode state of TileKVCache layers (or of a RetrievalIndex) saved to
and loaded from the versioned format of include/kvr_store.h, whose header codec, section
layout and CRC-32 live in libkvr_hip.so (host-only functions: they work without a GPU).

The reference has no such format: it keeps its store in device memory and rebuilds it on
reset (modules/kvr_hook.py:316-326, modules/kvr_retrieval.py:150-160).  A file written here
serves prefix caching (encode a long prompt once, load it for every request that shares it)
and the exchange of fixtures.

    save(f, caches, user=(...))          f: path or binary file object; caches: TileKVCache list
    load(f, device, reserve_tiles=...)   -> (caches, desc)
    to_bytes(caches) / from_bytes(buf, device)
    write_layers(f, desc, layers) / read_layers(f)   the format over plain arrays

Every cache of one file has the same batch, KV heads, tile size, transform, window size and
dtype, and the same window length and tile count (true of every layer of a KVRHook).  The
window is written oldest token first, so a loaded cache starts with its ring at slot 0; its
tile store is sized for n_tiles + reserve_tiles tiles.  Reading checks the header (magic,
version, header CRC, sizes) and the payload CRC-32 and raises ValueError on a mismatch or a
truncated file.
"""
from __future__ import annotations

import ctypes
import io
import os
import zlib

import numpy as np
import torch

from . import _hip

HEADER_BYTES = 256
FORMAT_VERSION = 1
HAS_COUNTS, HAS_WINDOW = 1, 2
BITS_TOKEN_LSB = 0
SEC_KBITS, SEC_VBITS, SEC_KSCALE, SEC_VSCALE, SEC_KCOUNT, SEC_WIN_K, SEC_WIN_V = range(7)
SECTIONS = (SEC_KBITS, SEC_VBITS, SEC_KSCALE, SEC_VSCALE, SEC_KCOUNT, SEC_WIN_K, SEC_WIN_V)
_WIN_NP = {_hip.BF16: np.uint16, _hip.FP16: np.float16, _hip.FP32: np.float32}


class StoreDesc(ctypes.Structure):
    """kvr_store_desc of include/kvr_store.h."""
    _fields_ = [("format_version", ctypes.c_uint32), ("abi_version", ctypes.c_uint32),
                ("d", ctypes.c_int32), ("T", ctypes.c_int32), ("transform", ctypes.c_int32),
                ("bit_order", ctypes.c_int32), ("scale_dtype", ctypes.c_int32), ("win_dtype", ctypes.c_int32),
                ("flags", ctypes.c_uint32), ("n_layers", ctypes.c_int32),
                ("B", ctypes.c_int64), ("Hkv", ctypes.c_int64), ("n_tiles", ctypes.c_int64),
                ("W", ctypes.c_int64), ("win_len", ctypes.c_int64),
                ("payload_bytes", ctypes.c_uint64), ("payload_crc32", ctypes.c_uint32),
                ("user", ctypes.c_int64 * 4)]

    def __repr__(self):
        return (f"StoreDesc(layers={self.n_layers}, B={self.B}, Hkv={self.Hkv}, T={self.T}, "
                f"transform={self.transform}, n_tiles={self.n_tiles}, W={self.W}, win_len={self.win_len}, "
                f"flags={self.flags}, payload={self.payload_bytes})")


def new_desc(*, T, transform, n_layers, B, Hkv, n_tiles, W=0, win_len=0, win_dtype=None, counts=True,
             user=(0, 0, 0, 0)) -> StoreDesc:
    d = StoreDesc()
    d.d, d.T, d.transform, d.bit_order, d.scale_dtype = 128, T, transform, BITS_TOKEN_LSB, _hip.FP16
    d.flags = (HAS_COUNTS if counts else 0) | (HAS_WINDOW if win_dtype is not None else 0)
    d.win_dtype = 0 if win_dtype is None else win_dtype
    d.n_layers, d.B, d.Hkv, d.n_tiles, d.W, d.win_len = n_layers, B, Hkv, n_tiles, W, win_len
    for i, u in enumerate(tuple(user)[:4]):
        d.user[i] = int(u)
    return d


def _check(rc, what):
    if rc < 0:
        raise ValueError(f"{what}: {_hip.last_error()} ({rc})")
    return rc


def payload_bytes(desc: StoreDesc) -> int:
    return _check(_hip.lib().kvr_store_payload_bytes(ctypes.byref(desc)), "kvr_store_payload_bytes")


def section(desc: StoreDesc, layer: int, sec: int):
    """(file offset, bytes) of one section (kvr_store_section)."""
    nbytes = ctypes.c_int64(0)
    off = _check(_hip.lib().kvr_store_section(ctypes.byref(desc), layer, sec, ctypes.byref(nbytes)),
                 "kvr_store_section")
    return off, nbytes.value


def present(desc: StoreDesc, sec: int) -> bool:
    if sec == SEC_KCOUNT:
        return bool(desc.flags & HAS_COUNTS)
    if sec in (SEC_WIN_K, SEC_WIN_V):
        return bool(desc.flags & HAS_WINDOW)
    return True


def encode_header(desc: StoreDesc) -> bytes:
    buf = ctypes.create_string_buffer(HEADER_BYTES)
    _check(_hip.lib().kvr_store_header_encode(ctypes.byref(desc), buf), "kvr_store_header_encode")
    return buf.raw


def decode_header(raw: bytes) -> StoreDesc:
    desc = StoreDesc()
    _check(_hip.lib().kvr_store_header_decode(raw, len(raw), ctypes.byref(desc)), "kvr_store_header_decode")
    return desc


def crc32(data, crc: int = 0) -> int:
    """kvr_crc32, the library's CRC-32 (the same function as zlib.crc32)."""
    raw = bytes(memoryview(data).cast("B"))
    return int(_hip.lib().kvr_crc32(crc, raw, len(raw)))


def section_shape(desc: StoreDesc, sec: int):
    """(numpy dtype, shape) of a section's array."""
    S, nt = desc.B * desc.Hkv, desc.n_tiles
    if sec in (SEC_KBITS, SEC_VBITS):
        return np.int64, (S, nt, 128, desc.T // 64)
    if sec in (SEC_KSCALE, SEC_VSCALE):
        return np.float16, (S, nt)
    if sec == SEC_KCOUNT:
        return np.uint8, (S, nt, 128)
    return _WIN_NP[desc.win_dtype], (desc.B, desc.Hkv, desc.win_len, 128)


def _host_bytes(x) -> bytes:
    if isinstance(x, torch.Tensor):
        x = x.detach().contiguous().cpu()
        return x.view(torch.uint8).numpy().tobytes() if x.numel() else b""
    return np.ascontiguousarray(x).tobytes()


def write_layers(f, desc: StoreDesc, layers) -> StoreDesc:
    """Write a store: layers[l][sec] = the section's array (torch tensor on any device, or
    numpy), in the dtype and shape of section_shape.  f: path or seekable binary file.
    Returns the description as written (payload size and CRC filled in)."""
    if len(layers) != desc.n_layers:
        raise ValueError(f"{len(layers)} layers for a description of {desc.n_layers}")
    own = isinstance(f, (str, os.PathLike))
    fh = open(f, "wb") if own else f
    try:
        base = fh.tell()
        fh.write(b"\0" * HEADER_BYTES)  # the header follows once the payload CRC is known
        pos, crc = HEADER_BYTES, 0
        for li, layer in enumerate(layers):
            for sec in SECTIONS:
                if not present(desc, sec):
                    continue
                off, nbytes = section(desc, li, sec)
                data = _host_bytes(layer[sec])
                if len(data) != nbytes:
                    raise ValueError(f"section {sec} of layer {li}: {len(data)} bytes, the layout needs {nbytes}")
                pad = b"\0" * (off - pos)
                fh.write(pad)
                fh.write(data)
                crc = zlib.crc32(data, zlib.crc32(pad, crc))
                pos = off + nbytes
        tail = b"\0" * (HEADER_BYTES + payload_bytes(desc) - pos)
        fh.write(tail)
        desc.payload_crc32 = zlib.crc32(tail, crc)
        header = encode_header(desc)
        end = fh.tell()
        fh.seek(base)
        fh.write(header)
        fh.seek(end)
    finally:
        if own:
            fh.close()
    return decode_header(header)


def _read_exact(fh, n):
    b = fh.read(n)
    if len(b) != n:
        raise ValueError(f"store file truncated: wanted {n} bytes, got {len(b)}")
    return b


def read_layers(f):
    """Read and verify a store -> (desc, layers) with layers[l][sec] a numpy array."""
    own = isinstance(f, (str, os.PathLike))
    fh = open(f, "rb") if own else f
    try:
        desc = decode_header(_read_exact(fh, HEADER_BYTES))
        layers, pos, crc = [], HEADER_BYTES, 0
        for li in range(desc.n_layers):
            layer = {}
            for sec in SECTIONS:
                if not present(desc, sec):
                    continue
                off, nbytes = section(desc, li, sec)
                pad = _read_exact(fh, off - pos)
                data = _read_exact(fh, nbytes)
                crc = zlib.crc32(data, zlib.crc32(pad, crc))
                pos = off + nbytes
                dt, shape = section_shape(desc, sec)
                layer[sec] = np.frombuffer(data, dtype=dt).reshape(shape)
            layers.append(layer)
        crc = zlib.crc32(_read_exact(fh, HEADER_BYTES + desc.payload_bytes - pos), crc)
        if crc != desc.payload_crc32:
            raise ValueError(f"store payload CRC mismatch (header {desc.payload_crc32:#010x}, data {crc:#010x}): "
                             "the file is corrupted")
    finally:
        if own:
            fh.close()
    return desc, layers


# ------------------------------------------------------------------ TileKVCache layers
def describe(caches, user=(0, 0, 0, 0)) -> StoreDesc:
    """The description of a list of TileKVCache layers (checks that they agree)."""
    if not caches:
        raise ValueError("nothing to save")
    c0 = caches[0]
    key = lambda c: (c.B, c.Hkv, c.T, c.transform, c.W, c.dtype, c.n, c.n_tiles)  # noqa: E731
    if any(key(c) != key(c0) for c in caches):
        raise ValueError("the caches of one store file must have the same shape and state")
    return new_desc(T=c0.T, transform=c0.transform, n_layers=len(caches), B=c0.B, Hkv=c0.Hkv, n_tiles=c0.n_tiles,
                    W=c0.W, win_len=c0.n, win_dtype=_hip._DT[c0.dtype], counts=True, user=user)


def save(f, caches, user=(0, 0, 0, 0)) -> StoreDesc:
    """Write TileKVCache layers (tiles, K channel counts and window) to f.  Copies every
    section to the host (synchronising with the device)."""
    desc = describe(caches, user)
    layers = []
    for c in caches:
        nt = c.n_tiles
        wk, wv = c.window_tokens()
        layers.append({SEC_KBITS: c.kbits[:, :nt], SEC_VBITS: c.vbits[:, :nt], SEC_KSCALE: c.kscale[:, :nt],
                       SEC_VSCALE: c.vscale[:, :nt], SEC_KCOUNT: c.kcount[:, :nt], SEC_WIN_K: wk, SEC_WIN_V: wv})
    return write_layers(f, desc, layers)


def counts_from_bits(bits: torch.Tensor) -> torch.Tensor:
    """uint8 [..., 128] set-bit counts per channel of int64 words [..., 128, T/64] (for
    stores written without the K channel counts)."""
    x = bits.contiguous().view(torch.uint8)
    table = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.uint8, device=bits.device)
    return table[x.long()].reshape(bits.shape + (8,)).sum(dim=(-1, -2), dtype=torch.int32).to(torch.uint8)


def load(f, device, reserve_tiles: int = 64, dtype=None):
    """Read a store into new TileKVCache layers on `device` -> (caches, desc).
    reserve_tiles: tile slots beyond the stored ones (decode steps add tiles); dtype: the
    window dtype of the new caches (default: the file's)."""
    from .kvr_cache import TileKVCache
    desc, layers = read_layers(f)
    if not desc.flags & HAS_WINDOW or desc.W < desc.T:
        raise ValueError("this store has no cache window (W=0): load it with RetrievalIndex.load_store")
    wdt = _hip._TORCH_DT[desc.win_dtype]
    nt, caches = desc.n_tiles, []
    for layer in layers:
        c = TileKVCache(desc.B, desc.Hkv, desc.W, desc.T, desc.transform, device, dtype or wdt,
                        tile_cap=nt + max(1, reserve_tiles))
        if nt:
            c.kbits[:, :nt] = torch.from_numpy(layer[SEC_KBITS].copy())
            c.vbits[:, :nt] = torch.from_numpy(layer[SEC_VBITS].copy())
            c.kscale[:, :nt] = torch.from_numpy(layer[SEC_KSCALE].copy())
            c.vscale[:, :nt] = torch.from_numpy(layer[SEC_VSCALE].copy())
            if SEC_KCOUNT in layer:
                c.kcount[:, :nt] = torch.from_numpy(layer[SEC_KCOUNT].copy())
            else:  # the decode step scores from the counts: rebuild them from the K bits
                c.kcount[:, :nt] = counts_from_bits(c.kbits[:, :nt])
        n = int(desc.win_len)
        if n:
            for sec, dst in ((SEC_WIN_K, c.win_k), (SEC_WIN_V, c.win_v)):
                dst[:, :, :n] = torch.from_numpy(layer[sec].copy()).view(wdt).to(c.dtype)
        c.n, c.start, c.n_tiles = n, 0, int(nt)
        c._push_state()
        caches.append(c)
    return caches, desc


def to_bytes(caches, **kw) -> bytes:
    buf = io.BytesIO()
    save(buf, caches, **kw)
    return buf.getvalue()


def from_bytes(raw: bytes, device, **kw):
    return load(io.BytesIO(raw), device, **kw)
