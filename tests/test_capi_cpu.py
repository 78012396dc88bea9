"""C-ABI checks that need no GPU: the library loads, exports exactly what include/*.h
(kvr_capi.h, kvr_store.h) declares, the ctypes signatures agree with the headers, and
host-side validation rejects bad arguments (every call here fails validation, so nothing is
launched)."""
import ctypes
import glob
import os
import re

import pytest

from conftest import REPO

HEADERS = sorted(glob.glob(os.path.join(REPO, "include", "*.h")))


@pytest.fixture(scope="module")
def H():
    from modules import _hip
    return _hip


@pytest.fixture(scope="module")
def lib(H):
    return H.lib()


def header_functions():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|uint32_t|size_t|const char\*)\s+(kvr_\w+)\s*\(([^;]*?)\)\s*;", text,
                         flags=re.S):
        args = m.group(2).strip()
        decls[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return decls


def test_library_exports_every_header_symbol(lib):
    decls = header_functions()
    assert len(HEADERS) == 2 and len(decls) >= 18
    for name in decls:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_ctypes_signatures_match_header(H):
    decls = header_functions()
    assert set(decls) == set(H.SIGNATURES)
    for name, nargs in decls.items():
        assert len(H.SIGNATURES[name][1]) == nargs, name


def test_abi_version(lib, H):
    assert lib.kvr_abi_version() == H.ABI_VERSION


FAKE = ctypes.c_void_p(0x10000)   # aligned, never dereferenced: validation fails first
FAKE_MIS = ctypes.c_void_p(0x10004)


def test_validation_errors_without_gpu(lib, H):
    # head_dim != 128
    assert lib.kvr_score_tiles(FAKE, FAKE, 1, 4, 4, 100, 64, None, None, 0, FAKE, None) == -1
    assert "head_dim" in H.last_error()
    # T not in {64, 128}
    assert lib.kvr_encode_tiles(FAKE, 0, 1, 1, 64, 0, 0, 128, 128, 32, 0, FAKE, FAKE, 2, 0, None, None, None) == -1
    # n_tok not a multiple of T
    assert lib.kvr_encode_tiles(FAKE, 0, 1, 1, 100, 0, 0, 128, 128, 64, 0, FAKE, FAKE, 2, 0, None, None, None) == -1
    assert "multiple" in H.last_error()
    # NONE transform needs fp32 input
    assert lib.kvr_encode_tiles(FAKE, 0, 1, 1, 64, 0, 0, 128, 128, 64, 2, FAKE, FAKE, 2, 0, None, None, None) == -1
    # tile slots beyond the store
    assert lib.kvr_encode_tiles(FAKE, 0, 1, 1, 128, 0, 0, 128, 128, 64, 0, FAKE, FAKE, 2, 1, None, None, None) == -1
    # misaligned input
    assert lib.kvr_encode_tiles(FAKE_MIS, 0, 1, 1, 64, 0, 0, 128, 128, 64, 0, FAKE, FAKE, 2, 0, None, None, None) == -2
    # top-k: k out of range
    assert lib.kvr_topk_tiles(FAKE, 1, 10, 10, 0, FAKE, None) == -1
    assert lib.kvr_topk_tiles(FAKE, 1, 10, 10, 11, FAKE, None) == -1
    assert lib.kvr_topk_tiles(FAKE, 1, 5000, 5000, 1025, FAKE, None) == -1
    # score: only one exclusion array
    assert lib.kvr_score_tiles(FAKE, FAKE, 1, 4, 4, 128, 64, FAKE, None, 0, FAKE, None) == -1
    # score: bad method
    assert lib.kvr_score_tiles(FAKE, FAKE, 1, 4, 4, 128, 64, None, None, 7, FAKE, None) == -1


def attn(lib, **kw):
    a = dict(q=FAKE, qdt=0, B=1, Hq=32, Hkv=8, d=128, wk=FAKE, wv=FAKE, wdt=0, wl=64, w0=0, wc=0, sb=0,
             sh=8192, st=128, kb=FAKE, vb=FAKE, ks=FAKE, vs=FAKE, ts=4, T=64, tf=0, idx=FAKE, k=2, out=FAKE,
             odt=2, ws=FAKE, wsb=0, s=None)
    a.update(kw)
    return lib.kvr_decode_attn(*a.values())


def test_decode_attn_validation(lib, H):
    assert attn(lib, Hq=30) == -1                      # Hq not a multiple of Hkv
    assert attn(lib, Hq=8 * 17) == -5                  # g > 16 not built
    assert "g=17" in H.last_error()
    assert attn(lib, odt=1) == -1                      # fp16 output not offered
    assert attn(lib, wdt=3) == -1                      # unknown window dtype
    assert attn(lib, wdt=2, st=126) == -2              # fp32 window: stride not a 16-byte multiple
    assert attn(lib, wdt=2) == -3                      # fp32 window accepted (fails at the workspace)
    assert attn(lib, st=100) == -2                     # window stride not 16-byte multiple
    assert attn(lib, wk=FAKE_MIS) == -2
    assert attn(lib, k=2000) == -1
    assert attn(lib, idx=None) == -1                   # k > 0 needs idx
    assert attn(lib, wc=32) == -1                      # win_len beyond the ring capacity
    assert "ring" in H.last_error()
    assert attn(lib, wc=128, w0=128) == -1             # ring start outside the ring
    assert attn(lib, w0=3) == -1                       # a start without a ring
    assert attn(lib, wsb=10) == -3                     # workspace too small
    need = lib.kvr_decode_attn_workspace(1, 32, 8, 64, 2, 64)
    assert attn(lib, wsb=need, ws=ctypes.c_void_p(0x10040)) == -2   # workspace misaligned


def step(lib, **kw):
    a = dict(q=FAKE, qdt=0, B=1, Hq=32, Hkv=8, d=128, wk=FAKE, wv=FAKE, wdt=0, wl=63, w0=0, wc=128, sb=0,
             sh=16384, st=128, kb=FAKE, vb=FAKE, ks=FAKE, vs=FAKE, kc=None, nt=8, ts=8, T=64, tf=0, lo=None,
             hi=None, k=2, live=FAKE, out=FAKE, odt=2, idx=None, ws=FAKE, wsb=0, s=None)
    a.update(kw)
    return lib.kvr_decode_step(*a.values())


def test_decode_step_live_validation(lib, H):
    assert step(lib, live=FAKE_MIS) == -2              # live state misaligned
    assert step(lib, wc=0) == -1                       # a live state needs a ring
    assert step(lib, k=65, nt=100, ts=100) == -5       # beyond the one-launch step
    assert "live state" in H.last_error()
    assert step(lib, k=9) == -1                        # k > tile capacity
    assert step(lib) == -3                             # otherwise valid: fails at the workspace


def append(lib, **kw):
    a = dict(k=FAKE, v=FAKE, ndt=0, B=1, Hkv=8, d=128, wk=FAKE, wv=FAKE, wdt=0, sb=0, sh=16384, st=128, W=64,
             T=64, tf=0, kb=FAKE, vb=FAKE, ks=FAKE, vs=FAKE, kc=None, ts=8, state=FAKE, s=None)
    a.update(kw)
    return lib.kvr_cache_append(*a.values())


def test_cache_append_validation(lib, H):
    assert append(lib, W=32) == -1                     # W not a multiple of T
    assert append(lib, W=0) == -1
    assert append(lib, tf=2) == -1                     # the cache encodes Hadamard or DCT
    assert append(lib, ndt=5) == -1
    assert append(lib, st=100) == -2                   # window stride
    assert append(lib, state=FAKE_MIS) == -2           # state alignment
    assert append(lib, state=None) == -1
    assert append(lib, ts=0) == -1                     # store pitch
    assert append(lib, B=0) == 0                       # nothing to do


def test_wait_limit_validation(lib):
    assert lib.kvr_set_wait_limit(-1, 0) == -1
    assert lib.kvr_set_wait_limit(0, 0) == 0           # restores the default


def test_workspace_sizes(lib):
    a = lib.kvr_decode_step_workspace(16, 32, 8, 1024, 496, 32, 64)
    b = lib.kvr_decode_step_workspace(16, 32, 8, 1024, 992, 32, 64)
    assert 0 < a < b
    assert lib.kvr_decode_attn_workspace(16, 32, 8, 1024, 32, 64) > 0
    assert lib.kvr_decode_step_workspace(1, 30, 8, 1024, 496, 32, 64) == 0   # invalid heads -> 0


def test_missing_library_fails_loudly(H, monkeypatch):
    monkeypatch.setattr(H, "_lib", None)
    monkeypatch.setattr(H, "LIB_PATH", "/nonexistent/libkvr_hip.so")
    with pytest.raises(RuntimeError, match="not built"):
        H.lib()


def test_cpu_tensors_are_rejected(H):
    import torch
    with pytest.raises(RuntimeError, match="device tensors"):
        H.encode_tiles(torch.zeros(1, 1, 64, 128), 64, H.HADAMARD)
