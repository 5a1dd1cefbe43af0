"""Packed weight layouts restated as reshape/transpose permutations.

The GPU pack (package csrc/pack.hip) computes the same permutation with
per-element index arithmetic; the tests require byte equality.  It replaces
the reference's mma.sync B-fragment pack (kernels/moe.cu:97-109,164-208),
which is a different layout by design (the packed format is private to the
forward, moe.cu:761-766).

W13 [E, 4096, 7168] -> [E, nb 16, kb 56, tile 16 (= 2*j + u), half 2, lane 64 (= 16*g + i), 16 B]
    source row = u*2048 + nb*128 + 16*j + i, source column = kb*128 + 32*g + 16*half + byte
W2  [E, 7168, 2048] -> [E, hb 56, kb 16, tile 8, half 2, lane 64, 16 B]
    source row = hb*128 + 16*tile + i,        source column = kb*128 + 32*g + 16*half + byte
"""

from __future__ import annotations

import numpy as np


def pack_w13(w13: np.ndarray) -> np.ndarray:
    E = w13.shape[0]
    # [E, u2, nb16, j8, i16, kb56, g4, h2, b16]
    v = w13.reshape(E, 2, 16, 8, 16, 56, 4, 2, 16)
    # -> [E, nb, kb, j, u, h, g, i, b]
    p = v.transpose(0, 2, 5, 3, 1, 7, 6, 4, 8)
    return np.ascontiguousarray(p).reshape(E, 16, 56, 16, 2, 64, 16)


def unpack_w13(packed: np.ndarray) -> np.ndarray:
    E = packed.shape[0]
    v = packed.reshape(E, 16, 56, 8, 2, 2, 4, 16, 16)  # [E, nb, kb, j, u, h, g, i, b]
    w = v.transpose(0, 4, 1, 3, 7, 2, 6, 5, 8)         # -> [E, u, nb, j, i, kb, g, h, b]
    return np.ascontiguousarray(w).reshape(E, 4096, 7168)


def pack_w2(w2: np.ndarray) -> np.ndarray:
    E = w2.shape[0]
    # [E, hb56, t8, i16, kb16, g4, h2, b16]
    v = w2.reshape(E, 56, 8, 16, 16, 4, 2, 16)
    # -> [E, hb, kb, t, h, g, i, b]
    p = v.transpose(0, 1, 4, 2, 6, 5, 3, 7)
    return np.ascontiguousarray(p).reshape(E, 56, 16, 8, 2, 64, 16)


def unpack_w2(packed: np.ndarray) -> np.ndarray:
    E = packed.shape[0]
    v = packed.reshape(E, 56, 16, 8, 2, 4, 16, 16)   # [E, hb, kb, t, h, g, i, b]
    w = v.transpose(0, 1, 3, 6, 2, 5, 4, 7)          # -> [E, hb, t, i, kb, g, h, b]
    return np.ascontiguousarray(w).reshape(E, 7168, 2048)
