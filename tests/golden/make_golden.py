"""Writes the golden fixtures of this directory (tests/golden/golden_*.npz) from the CPU oracle.

The reference has no tests, golden vectors or fixtures for this path, so these fixtures are
regression anchors of this build: fixed seeded inputs (rebuilt from the seed by `inputs()`,
with a checksum stored to catch generator drift) and the oracle's outputs for them -- packed
bits and fp16 scales of K and V, the rotated GQA-mean query, tile scores, the top-k tile
indices and the float64 decode attention output.  The oracle functions they come from are
pinned by the known-answer, closed-form and brute-force tests of tests/test_oracle.py.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))
from oracle import kvr_oracle as O  # noqa: E402

# name -> (T, transform, seed); B = 1, Hq = 8, Hkv = 2, 3 tiles, window 32, top-2 tiles
CASES = {"hadamard_t64": (64, O.HADAMARD, 11), "dct_t128": (128, O.DCT, 12)}
B, HQ, HKV, N_TILES, W, K_SEL = 1, 8, 2, 3, 32, 2


def inputs(T, seed):
    """bf16-exact fp32 inputs: K (log-normal channel scales) and V [S, n_tok, 128], q [B, Hq, 128],
    window K/V [B, Hkv, W, 128]."""
    rng = np.random.default_rng(seed)
    S = B * HKV
    ch = np.exp(rng.normal(0.0, 1.0, 128)).astype(np.float32)
    K = O.bf16_round(rng.standard_normal((S, N_TILES * T, 128)).astype(np.float32) * ch)
    V = O.bf16_round(rng.standard_normal((S, N_TILES * T, 128)).astype(np.float32))
    q = O.bf16_round(rng.standard_normal((B, HQ, 128)).astype(np.float32))
    win_k = O.bf16_round(rng.standard_normal((B, HKV, W, 128)).astype(np.float32) * ch)
    win_v = O.bf16_round(rng.standard_normal((B, HKV, W, 128)).astype(np.float32))
    return K, V, q, win_k, win_v


def checksum(*arrays):
    return np.uint64(sum(int(O.bf16_to_bits(a).astype(np.uint64).sum()) for a in arrays))


def outputs(T, tf, seed):
    K, V, q, win_k, win_v = inputs(T, seed)
    kbits, kscale = O.encode(K, T, tf)
    vbits, vscale = O.encode(V, T, tf)
    qbar, _ = O.query_prep(q, HKV, tf)
    scores = O.score_tiles(qbar.reshape(-1, 128), kbits)
    idx = O.topk_tiles(scores, K_SEL)
    out = O.decode_attention(q, win_k, win_v, kbits, vbits, kscale, vscale, idx, tf)
    return dict(T=T, transform=tf, seed=seed, input_checksum=checksum(K, V, q, win_k, win_v),
                kbits=kbits, kscale=kscale, vbits=vbits, vscale=vscale, qbar=qbar.reshape(-1, 128),
                scores=scores, idx=idx, out=out)


def main():
    for name, (T, tf, seed) in CASES.items():
        path = os.path.join(HERE, f"golden_{name}.npz")
        np.savez_compressed(path, **outputs(T, tf, seed))
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
