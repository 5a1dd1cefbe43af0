"""Upstream producer of the forward's inputs -- TEST INFRASTRUCTURE ONLY.

The forward consumes router logits f32 [T,256] and block-scaled FP8
activations (e4m3 [T,7168] + scale f32 [56,T], block-major as in
reference/moe_ref.py:49,60-61).  The reference has no producer for them (its
builder draws random ones, moe_layer.py:45-75); this module restates the
producer the build adds in front of the path:

  logits[t, e]      = sum_h x[t, h] * w[e, h]      bf16 x and w, exact products
  scale[kb, t]      = max(amax(|x[t, kb*128 : kb*128+128]|) / 448, 1e-8)   (fp32)
  hidden_fp8[t, h]  = e4m3_rne(clamp(x[t, h] / scale, -448, 448))         (fp32 divide)

The quantisation is the path's own requant formula (kernels/moe.cu:516-541,
applied there to the SwiGLU output), so one rule covers both FP8 producers.

Pinning: `act_quant` is bit-exact against the GPU kernel and is fixed by
known answers (the block maximum maps to +-448 = code 0x7E, zero blocks give
scale 1e-8 and zero codes, a block of equal magnitudes gives one code) and
the dequantisation round trip (|x - decode(code)*scale| <= half an e4m3 step
of x); `router_logits` sums the exact bf16 products in float64 (error about
1e-16 of sum|x*w|, far below the fp32 accumulation error it checks) and is
fixed by one-hot rows that select single weights; `pack_router` is
byte-equal to the GPU pack and inverted by `unpack_router`
(tests/test_upstream.py).
"""

from __future__ import annotations

import numpy as np

from .numerics import bf16_value, e4m3_encode

H = 7168
E_GLOBAL = 256
BLOCK = 128


def act_quant(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """bf16 bits [T, 7168] -> (codes u8 [T, 7168], scale f32 [56, T])."""
    x = bf16_value(x_bits).reshape(-1, H // BLOCK, BLOCK)              # fp32, exact
    T = x.shape[0]
    amax = np.abs(x).max(axis=2)                                       # [T, 56]
    scale = np.maximum((amax / np.float32(448.0)).astype(np.float32), np.float32(1e-8)).astype(np.float32)
    q = (x / scale[:, :, None]).astype(np.float32)
    q = np.clip(q, np.float32(-448.0), np.float32(448.0))
    return e4m3_encode(q.reshape(T, H)), np.ascontiguousarray(scale.T)


def router_logits(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """bf16 bits x [T, 7168], w [256, 7168] -> float64 [T, 256] (exact sums)."""
    x = bf16_value(x_bits).astype(np.float64)
    w = bf16_value(w_bits).astype(np.float64)
    return x @ w.T


def logits_bound(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """sum_h |x*w| per (t, e): the scale of an fp32 accumulation error."""
    x = np.abs(bf16_value(x_bits).astype(np.float64))
    w = np.abs(bf16_value(w_bits).astype(np.float64))
    return x @ w.T


# Packed router weight (the GPU kernel's MFMA A-operand layout for
# v_mfma_f32_16x16x32_bf16): [kb 56][ks 4][expert tile 16][lane 64][8 bf16],
# lane l = 16*g + i holds expert 16*tile + i, K = kb*128 + ks*32 + 8*g .. +8.
def pack_router(w_bits: np.ndarray) -> np.ndarray:
    v = np.asarray(w_bits, dtype=np.uint16).reshape(16, 16, 56, 4, 4, 8)  # [tile, i, kb, ks, g, e8]
    p = v.transpose(2, 3, 0, 4, 1, 5)                                     # [kb, ks, tile, g, i, e8]
    return np.ascontiguousarray(p).reshape(56, 4, 16, 64, 8)


def unpack_router(packed: np.ndarray) -> np.ndarray:
    v = np.asarray(packed, dtype=np.uint16).reshape(56, 4, 16, 4, 16, 8)  # [kb, ks, tile, g, i, e8]
    w = v.transpose(2, 4, 0, 1, 3, 5)                                     # [tile, i, kb, ks, g, e8]
    return np.ascontiguousarray(w).reshape(E_GLOBAL, H)
