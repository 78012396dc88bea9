"""Writes tests/golden/store_v1_hadamard_t64.kvrs: a one-layer tile-store file (format
version 1 of include/kvr_store.h) holding the oracle's encoding of a seeded input, as a
regression anchor of the on-disk format (the reference has no store format to compare
with).  Run from the repository root:  python tests/golden/make_store_golden.py

Content: B=1, Hkv=1, T=64, Hadamard; tokens 0..127 (two tiles, K channel counts included)
and a bf16 window of the next 66 tokens (W=64), user words (194, 7, 0, 0).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (REPO, os.path.join(REPO, "rina-1bit-kv_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import kvr_oracle as O  # noqa: E402

PATH = os.path.join(HERE, "store_v1_hadamard_t64.kvrs")
SEED, T, N_TILES, W, WIN_LEN = 11, 64, 2, 64, 66
USER = (194, 7, 0, 0)


def golden_input():
    """(k, v) fp32 [1, n, 128] rounded to bf16, n = N_TILES * T + WIN_LEN."""
    g = np.random.default_rng(SEED)
    n = N_TILES * T + WIN_LEN
    k = g.standard_normal((1, n, 128)).astype(np.float32) * np.exp(g.standard_normal(128)).astype(np.float32)
    v = g.standard_normal((1, n, 128)).astype(np.float32)
    return O.bf16_round(k), O.bf16_round(v)


def golden_sections():
    """The section arrays of the golden store (oracle encoding)."""
    from modules import kvr_store as S
    k, v = golden_input()
    nr = N_TILES * T
    kb, ks = O.encode(k[:, :nr], T, O.HADAMARD)
    vb, vs = O.encode(v[:, :nr], T, O.HADAMARD)
    counts = np.unpackbits(kb.view(np.uint8), axis=-1).reshape(kb.shape + (64,)).sum(axis=(-1, -2))
    return {S.SEC_KBITS: kb.view(np.int64), S.SEC_VBITS: vb.view(np.int64), S.SEC_KSCALE: ks,
            S.SEC_VSCALE: vs, S.SEC_KCOUNT: counts.astype(np.uint8),
            S.SEC_WIN_K: O.bf16_to_bits(k[:, nr:]).reshape(1, 1, WIN_LEN, 128),
            S.SEC_WIN_V: O.bf16_to_bits(v[:, nr:]).reshape(1, 1, WIN_LEN, 128)}


def golden_desc():
    from modules import _hip
    from modules import kvr_store as S
    return S.new_desc(T=T, transform=_hip.HADAMARD, n_layers=1, B=1, Hkv=1, n_tiles=N_TILES, W=W,
                      win_len=WIN_LEN, win_dtype=_hip.BF16, counts=True, user=USER)


def main():
    from modules import kvr_store as S
    desc = S.write_layers(PATH, golden_desc(), [golden_sections()])
    print(f"wrote {PATH}: {os.path.getsize(PATH)} bytes, {desc}")


if __name__ == "__main__":
    main()
