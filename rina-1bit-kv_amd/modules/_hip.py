"""ctypes binding of libkvr_hip.so (the C ABI in include/kvr_capi.h).

The HIP library is the only implementation of the hot path: if it is missing or
no GPU is present these functions raise; there is no CPU fallback.  Tensors are
PyTorch-ROCm device tensors used as plain memory; every call is launched on
torch's current stream and returns without synchronising.
"""
from __future__ import annotations

import ctypes
import os

import torch

BF16, FP16, FP32 = 0, 1, 2
HADAMARD, DCT, NONE = 0, 1, 2
TRANSFORMS = {"hadamard": HADAMARD, "dct": DCT, "none": NONE}
_DT = {torch.bfloat16: BF16, torch.float16: FP16, torch.float32: FP32}
_TORCH_DT = {BF16: torch.bfloat16, FP16: torch.float16, FP32: torch.float32}

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkvr_hip.so")
ABI_VERSION = 4

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_Z = ctypes.c_size_t

# name -> (restype, argtypes); the single source of the Python-side signatures.
SIGNATURES = {
    "kvr_abi_version": (_I, []),
    "kvr_last_error": (ctypes.c_char_p, []),
    "kvr_encode_tiles": (_I, [_P, _I, _L, _L, _L, _L, _L, _L, _I, _I, _I, _P, _P, _L, _L, _P, _P, _P]),
    "kvr_query_prep": (_I, [_P, _I, _L, _I, _I, _I, _I, _P, _P, _P]),
    "kvr_score_tiles": (_I, [_P, _P, _L, _L, _L, _I, _I, _P, _P, _I, _P, _P]),
    "kvr_topk_tiles": (_I, [_P, _L, _L, _L, _I, _P, _P]),
    "kvr_decode_attn_workspace": (_Z, [_L, _I, _I, _L, _I, _I]),
    "kvr_decode_attn": (_I, [_P, _I, _L, _I, _I, _I, _P, _P, _I, _L, _L, _L, _L, _L, _L, _P, _P, _P, _P,
                             _L, _I, _I, _P, _I, _P, _I, _P, _Z, _P]),
    "kvr_decode_step_workspace": (_Z, [_L, _I, _I, _L, _L, _I, _I]),
    "kvr_decode_step": (_I, [_P, _I, _L, _I, _I, _I, _P, _P, _I, _L, _L, _L, _L, _L, _L, _P, _P, _P, _P, _P,
                             _L, _L, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _Z, _P]),
    "kvr_gather_tiles": (_I, [_P, _P, _L, _L, _I, _I, _P, _I, _P, _L, _L, _P]),
    "kvr_cache_append": (_I, [_P, _P, _I, _L, _I, _I, _P, _P, _I, _L, _L, _L, _L, _I, _I, _P, _P, _P, _P, _P,
                              _L, _P, _P]),
    "kvr_set_wait_limit": (_I, [_I, _I]),
    "kvr_decode_step_noalloc": (_I, [_P, _I, _L, _I, _I, _I, _P, _P, _I, _L, _L, _L, _L, _L, _L, _P, _P, _P, _P,
                                     _P, _L, _L, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P]),
    # tile-store format (include/kvr_store.h): host-only, callable without a GPU
    "kvr_crc32": (ctypes.c_uint32, [ctypes.c_uint32, _P, _Z]),
    "kvr_store_payload_bytes": (_L, [_P]),
    "kvr_store_section": (_L, [_P, _I, _I, _P]),
    "kvr_store_header_encode": (_I, [_P, _P]),
    "kvr_store_header_decode": (_I, [_P, _Z, _P]),
}

_lib = None


def lib():
    """Load libkvr_hip.so once (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `make -C rina-1bit-kv_amd/csrc` or "
                "`python -c 'import __graft_entry__ as g; g.build()'` (no CPU fallback exists)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.kvr_abi_version() != ABI_VERSION:
            raise RuntimeError("libkvr_hip.so ABI version mismatch; rebuild it")
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().kvr_last_error().decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("kvr HIP kernels need device tensors (no CPU fallback)")


def tiles_words(T: int) -> int:
    return T // 64


def alloc_store(n_seg: int, tile_cap: int, T: int, device) -> tuple:
    """(bits int64 [n_seg, tile_cap, 128, T/64], scales fp16 [n_seg, tile_cap]) zero-filled."""
    bits = torch.zeros((n_seg, tile_cap, 128, T // 64), dtype=torch.int64, device=device)
    scales = torch.zeros((n_seg, tile_cap), dtype=torch.float16, device=device)
    return bits, scales


def alloc_counts(n_seg: int, tile_cap: int, device) -> torch.Tensor:
    """Per-tile channel counts of a K store, uint8 [n_seg, tile_cap, 128], zero-filled: entry
    (s, i, j) is the number of set bits of channel j over tile i's T tokens (2*count - T is
    the tile's column sum, all a tile score reads)."""
    return torch.zeros((n_seg, tile_cap, 128), dtype=torch.uint8, device=device)


# ----------------------------------------------------------------------------- encode

def encode_tiles(x: torch.Tensor, T: int, transform: int, bits=None, scales=None, tile_offset: int = 0,
                 want_rotated: bool = False, counts=None):
    """Encode x [n_b, n_h, n_tok, 128] (last dim contiguous, any other strides) into 1-bit tiles.

    Writes tiles [tile_offset, tile_offset + n_tok/T) of each segment b*n_h+h of the store
    (bits [n_b*n_h, cap, 128, T/64] int64, scales [n_b*n_h, cap] fp16), allocating a
    store of exactly n_tok/T tiles when none is given.  counts (optional, alloc_counts
    [n_b*n_h, cap, 128] uint8) receives the same tiles' channel counts.  Returns
    (bits, scales[, rotated]).
    """
    _require_gpu(x)
    if x.dim() != 4 or x.shape[-1] != 128 or x.stride(-1) != 1:
        raise ValueError("x must be [n_b, n_h, n_tok, 128] with a contiguous last dim")
    n_b, n_h, n_tok, _ = x.shape
    if n_tok % T:
        raise ValueError(f"n_tok={n_tok} is not a multiple of T={T}")
    n_tiles = n_tok // T
    if bits is None:
        bits, scales = alloc_store(n_b * n_h, tile_offset + n_tiles, T, x.device)
    rot = torch.empty((n_b * n_h, n_tok, 128), dtype=torch.float32, device=x.device) if want_rotated else None
    if counts is not None and (counts.dtype != torch.uint8 or tuple(counts.shape) != (bits.shape[0], bits.shape[1], 128)
                               or not counts.is_contiguous()):
        raise ValueError("counts must be a contiguous uint8 [n_seg, tile_cap, 128] tensor matching the store")
    sb, sh, st, _ = x.stride()
    rc = lib().kvr_encode_tiles(_ptr(x), _DT[x.dtype], n_b, n_h, n_tok, sb, sh, st, 128, T, transform,
                                _ptr(bits), _ptr(scales), bits.shape[1], tile_offset, _ptr(rot), _ptr(counts),
                                _stream())
    check(rc, "kvr_encode_tiles")
    return (bits, scales, rot) if want_rotated else (bits, scales)


# ----------------------------------------------------------------------------- query / score / top-k

def query_prep(q: torch.Tensor, n_kv: int, transform: int, want_q_rot: bool = True):
    """q [B, Hq, 128] -> (qbar_rot [B*Hkv, 128] fp32, q_rot [B*Hq, 128] fp32 or None)."""
    _require_gpu(q)
    q = q.contiguous()
    B, Hq, _ = q.shape
    qbar = torch.empty((B * n_kv, 128), dtype=torch.float32, device=q.device)
    qrot = torch.empty((B * Hq, 128), dtype=torch.float32, device=q.device) if want_q_rot else None
    rc = lib().kvr_query_prep(_ptr(q), _DT[q.dtype], B, Hq, n_kv, 128, transform, _ptr(qbar), _ptr(qrot),
                              _stream())
    check(rc, "kvr_query_prep")
    return qbar, qrot


def score_tiles(qbar_rot: torch.Tensor, kbits: torch.Tensor, n_tiles: int, T: int, excl_lo=None,
                excl_hi=None, method: int = 0, out=None):
    """Scores [BH, n_tiles] fp32 of the first n_tiles tiles of each segment."""
    _require_gpu(qbar_rot, kbits)
    BH = kbits.shape[0]
    if out is None:
        out = torch.empty((BH, n_tiles), dtype=torch.float32, device=kbits.device)
    rc = lib().kvr_score_tiles(_ptr(qbar_rot.contiguous()), _ptr(kbits), BH, n_tiles, kbits.shape[1], 128,
                               T, _ptr(excl_lo), _ptr(excl_hi), method, _ptr(out), _stream())
    check(rc, "kvr_score_tiles")
    return out


def topk_tiles(scores: torch.Tensor, k: int, out=None):
    """idx [BH, k] int32: score descending, ties by tile index ascending."""
    _require_gpu(scores)
    BH, n = scores.shape
    if out is None:
        out = torch.empty((BH, k), dtype=torch.int32, device=scores.device)
    rc = lib().kvr_topk_tiles(_ptr(scores), BH, n, scores.stride(0), k, _ptr(out), _stream())
    check(rc, "kvr_topk_tiles")
    return out


# ----------------------------------------------------------------------------- attention

def _window_args(win_k, win_v, win_len, win_start=0, win_cap=0):
    if win_k is None or (win_len == 0 and win_cap == 0):
        return None, None, BF16, 0, 0, 0, 0, 0, 0
    if win_k.stride() != win_v.stride() or win_k.stride(-1) != 1:
        raise ValueError("window K and V need identical strides and a contiguous last dim")
    sb, sh, st, _ = win_k.stride()
    return win_k, win_v, _DT[win_k.dtype], win_len, win_start, win_cap, sb, sh, st


def decode_attn(q, win_k, win_v, win_len, kbits, vbits, kscale, vscale, idx, T, transform,
                out_dtype=torch.float32, workspace=None, win_start=0, win_cap=0):
    """Fused window + retrieved-tile attention.  q [B, Hq, 128]; window [B, Hkv, slots, 128]
    (tokens in slots [0, win_len), or a ring of win_cap slots from win_start)."""
    _require_gpu(q, win_k, kbits, idx)
    q = q.contiguous()
    B, Hq, _ = q.shape
    Hkv = win_k.shape[1] if win_k is not None else kbits.shape[0] // B
    k = 0 if idx is None else idx.shape[1]
    wk, wv, wdt, wl, w0, wc, sb, sh, st = _window_args(win_k, win_v, win_len, win_start, win_cap)
    need = lib().kvr_decode_attn_workspace(B, Hq, Hkv, wl, k, T)
    if workspace is None or workspace.numel() < need:
        workspace = torch.zeros(max(need, 256), dtype=torch.uint8, device=q.device)  # zeroed counter region
    out = torch.empty((B, Hq, 128), dtype=out_dtype, device=q.device)
    tile_stride = kbits.shape[1] if kbits is not None else 1
    rc = lib().kvr_decode_attn(_ptr(q), _DT[q.dtype], B, Hq, Hkv, 128, _ptr(wk), _ptr(wv), wdt, wl, w0, wc,
                               sb, sh, st, _ptr(kbits), _ptr(vbits), _ptr(kscale), _ptr(vscale), tile_stride, T,
                               transform, _ptr(idx), k, _ptr(out), _DT[out_dtype], _ptr(workspace),
                               workspace.numel(), _stream())
    check(rc, "kvr_decode_attn")
    return out


COUNTER_BYTES = 256 + 2 * 4096 * 128  # counter region at the start of every decode workspace


def decode_step_workspace(B, Hq, Hkv, win_len, n_tiles, k, T, device):
    """Workspace for decode_step / decode_attn, zeroed: it begins with the launch's counter
    region (COUNTER_BYTES; int32 word 0 is a sticky error word), which the calls keep from one
    call to the next; the rest is scratch.  Reuse one workspace across calls on one stream,
    one per concurrent stream."""
    need = lib().kvr_decode_step_workspace(B, Hq, Hkv, win_len, n_tiles, k, T)
    return torch.zeros(max(need, 256), dtype=torch.uint8, device=device)


def decode_step(q, win_k, win_v, win_len, kbits, vbits, kscale, vscale, n_tiles, T, transform, k,
                excl_lo=None, excl_hi=None, out_dtype=torch.bfloat16, out=None, idx_out=None,
                workspace=None, kcounts=None, win_start=0, win_cap=0, live_state=None):
    """The whole decode hot path for one layer (query prep, scoring, top-k, attention).
    kcounts (optional): the K store's channel counts (alloc_counts, written by encode_tiles);
    tiles are then scored from them, with the same scores.  A ring window: win_cap slots,
    tokens from win_start on.  live_state (optional, int32 [B*Hkv, 4] device tensor as
    cache_append keeps it): the kernel reads each segment's window length, ring start and
    tile count from it, and win_len / n_tiles are the capacities."""
    if kcounts is not None and (kcounts.dtype != torch.uint8 or kbits is None
                                or tuple(kcounts.shape) != (kbits.shape[0], kbits.shape[1], 128)
                                or not kcounts.is_contiguous()):
        raise ValueError("kcounts must be a contiguous uint8 [n_seg, tile_cap, 128] tensor matching kbits")
    _require_gpu(q)
    q = q.contiguous()
    B, Hq, _ = q.shape
    Hkv = win_k.shape[1] if win_k is not None else kbits.shape[0] // B
    if live_state is not None:
        _check_state(live_state, B * Hkv)
    wk, wv, wdt, wl, w0, wc, sb, sh, st = _window_args(win_k, win_v, win_len, win_start, win_cap)
    if workspace is None:
        workspace = decode_step_workspace(B, Hq, Hkv, wl, n_tiles, k, T, q.device)
    if out is None:
        out = torch.empty((B, Hq, 128), dtype=out_dtype, device=q.device)
    tile_stride = kbits.shape[1] if kbits is not None else 1
    rc = lib().kvr_decode_step(_ptr(q), _DT[q.dtype], B, Hq, Hkv, 128, _ptr(wk), _ptr(wv), wdt, wl, w0, wc,
                               sb, sh, st, _ptr(kbits), _ptr(vbits), _ptr(kscale), _ptr(vscale), _ptr(kcounts),
                               n_tiles, tile_stride, T, transform, _ptr(excl_lo), _ptr(excl_hi), k,
                               _ptr(live_state), _ptr(out), _DT[out.dtype], _ptr(idx_out), _ptr(workspace),
                               workspace.numel(), _stream())
    check(rc, "kvr_decode_step")
    return out


NOALLOC_SCRATCH_BYTES = 16 << 20  # KVR_NOALLOC_SCRATCH_BYTES


def decode_step_noalloc(q, win_k, win_v, win_len, kbits, vbits, kscale, vscale, n_tiles, T, transform, k,
                        excl_lo=None, excl_hi=None, out_dtype=torch.bfloat16, out=None, idx_out=None,
                        kcounts=None, win_start=0, win_cap=0, live_state=None):
    """decode_step through kvr_decode_step_noalloc: no workspace (the library's per-GPU
    scratch); the output (and idx_out) are the caller's."""
    _require_gpu(q)
    q = q.contiguous()
    B, Hq, _ = q.shape
    Hkv = win_k.shape[1] if win_k is not None else kbits.shape[0] // B
    if live_state is not None:
        _check_state(live_state, B * Hkv)
    wk, wv, wdt, wl, w0, wc, sb, sh, st = _window_args(win_k, win_v, win_len, win_start, win_cap)
    if out is None:
        out = torch.empty((B, Hq, 128), dtype=out_dtype, device=q.device)
    tile_stride = kbits.shape[1] if kbits is not None else 1
    rc = lib().kvr_decode_step_noalloc(_ptr(q), _DT[q.dtype], B, Hq, Hkv, 128, _ptr(wk), _ptr(wv), wdt, wl, w0, wc,
                                       sb, sh, st, _ptr(kbits), _ptr(vbits), _ptr(kscale), _ptr(vscale),
                                       _ptr(kcounts), n_tiles, tile_stride, T, transform, _ptr(excl_lo),
                                       _ptr(excl_hi), k, _ptr(live_state), _ptr(out), _DT[out.dtype], _ptr(idx_out),
                                       _stream())
    check(rc, "kvr_decode_step_noalloc")
    return out


def workspace_status(workspace) -> int:
    """The workspace's sticky status word (int32 at byte 0; synchronises with the device):
    nonzero once a bounded wait of a decode step gave up."""
    return int(workspace[:4].view(torch.int32).item())


def check_workspace(workspace, what="decode step"):
    """Raise RuntimeError if a decode step on this workspace gave up a bounded wait; the
    workspace is zeroed again first, so it is usable afterwards."""
    st = workspace_status(workspace)
    if st != 0:
        workspace.zero_()
        raise RuntimeError(f"{what}: a bounded wait gave up (workspace status {st}); the outputs of the calls "
                           "since the workspace was last zeroed are unreliable (affected ones are NaN)")


def set_wait_limit(polls: int = 0, force_give_up: bool = False) -> None:
    """Bounded-wait polls of later decode launches (0 = default) and the diagnostic switch
    that makes the one-launch step's waits give up (tests of the failure path)."""
    check(lib().kvr_set_wait_limit(int(polls), int(bool(force_give_up))), "kvr_set_wait_limit")


# ----------------------------------------------------------------------------- ring cache append

STATE_WORDS = 4  # per segment: n (window tokens), start (ring slot), n_tiles, error


def _check_state(state, n_seg):
    if (state.dtype != torch.int32 or tuple(state.shape) != (n_seg, STATE_WORDS) or not state.is_contiguous()
            or not state.is_cuda):
        raise ValueError(f"state must be a contiguous int32 [{n_seg}, {STATE_WORDS}] device tensor")


def cache_append(k_new, v_new, win_k, win_v, W, T, transform, kbits, vbits, kscale, vscale, kcounts, state):
    """One token per segment (k_new, v_new [B, Hkv, 128]) into a ring window [B, Hkv, W + T, 128]
    and, when the ring fills, its oldest T tokens into the next tile slot; state is the
    int32 [B*Hkv, 4] device tensor {n, start, n_tiles, error} the kernel keeps."""
    _require_gpu(k_new, v_new, win_k, kbits, state)
    k_new = k_new.contiguous()
    v_new = v_new.to(k_new.dtype).contiguous()
    B, Hkv, _ = k_new.shape
    _check_state(state, B * Hkv)
    if win_k.shape[2] != W + T or win_k.stride() != win_v.stride() or win_k.stride(-1) != 1:
        raise ValueError("the ring window must be [B, Hkv, W + T, 128] with K and V strides equal")
    if kcounts is not None and tuple(kcounts.shape) != (kbits.shape[0], kbits.shape[1], 128):
        raise ValueError("kcounts must match the store")
    sb, sh, st, _ = win_k.stride()
    rc = lib().kvr_cache_append(_ptr(k_new), _ptr(v_new), _DT[k_new.dtype], B, Hkv, 128, _ptr(win_k), _ptr(win_v),
                                _DT[win_k.dtype], sb, sh, st, W, T, transform, _ptr(kbits), _ptr(vbits),
                                _ptr(kscale), _ptr(vscale), _ptr(kcounts), kbits.shape[1], _ptr(state), _stream())
    check(rc, "kvr_cache_append")


def gather_tiles(bits, scales, idx, T, transform, out=None):
    """Tokens of the selected tiles in the original domain: [BH, k*T, 128] fp32."""
    _require_gpu(bits, idx)
    BH, k = idx.shape
    if out is None:
        out = torch.empty((BH, k * T, 128), dtype=torch.float32, device=bits.device)
    rc = lib().kvr_gather_tiles(_ptr(bits), _ptr(scales), BH, bits.shape[1], T, transform, _ptr(idx), k,
                                _ptr(out), out.stride(0), out.stride(1), _stream())
    check(rc, "kvr_gather_tiles")
    return out
