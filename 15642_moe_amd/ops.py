"""Host-side mirror of the reference's ``ops`` module (pybind11 ``moe_fused``,
kernels/moe.cu:902-909): ``pack_w13``, ``pack_w2`` and ``moe_forward`` with the
reference's argument order, shape/dtype checks and RuntimeError behaviour,
implemented over the C ABI (include/moe_fp8.h).

Every function runs asynchronously on the current HIP stream of the input's
device.  There is no CPU path: CPU tensors raise RuntimeError.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import capi
from .geometry import (
    E_GLOBAL,
    G1_BLOCKS,
    H,
    H_BLOCKS,
    I_BLOCKS,
    I_DIM,
    MAX_E_LOCAL,
    TOP_K,
    W13_PACKED_SHAPE,
    W2_PACKED_SHAPE,
)


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_device(name: str, t: torch.Tensor, device: torch.device | None = None) -> None:
    _check(t.is_cuda, f"{name} must be a HIP device tensor (no CPU path)")
    if device is not None:
        _check(t.device == device, f"{name} must be on {device}, got {t.device}")


# --------------------------------------------------------------------------- packs
def _check_out(out: torch.Tensor | None, shape: tuple, like: torch.Tensor, name: str) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=torch.int32, device=like.device)
    _check(out.dtype == torch.int32 and tuple(out.shape) == shape and out.is_contiguous(),
           f"{name} out must be int32 {list(shape)} contiguous")
    _require_device(f"{name} out", out, like.device)
    return out


def pack_w13(W13: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """W13 e4m3 [E_local, 4096, 7168] -> int32 packed MFMA operand tiles
    (kernels/moe.cu:700-720).  `out` (optional) receives them in place, e.g.
    one expert's slot ``packed[e:e+1]`` of a larger packed buffer."""
    _require_device("W13", W13)
    _check(W13.dim() == 3, "W13 must be [E_local, 4096, 7168]")
    _check(W13.element_size() == 1, "W13 must be an FP8 tensor")
    _check(W13.is_contiguous(), "W13 must be contiguous")
    E = int(W13.size(0))
    _check(W13.size(1) == 2 * I_DIM and W13.size(2) == H, "W13 must be [E_local, 4096, 7168]")
    out = _check_out(out, (E, *W13_PACKED_SHAPE), W13, "pack_w13")
    if E == 0:
        return out
    with torch.cuda.device(W13.device):
        capi.check(capi.load().moe_pack_w13(_ptr(W13), _ptr(out), E, _stream(W13.device)), "pack_w13")
    return out


def pack_w2(W2: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """W2 e4m3 [E_local, 7168, 2048] -> int32 packed MFMA operand tiles
    (kernels/moe.cu:722-742); `out` as for pack_w13."""
    _require_device("W2", W2)
    _check(W2.dim() == 3, "W2 must be [E_local, 7168, 2048]")
    _check(W2.element_size() == 1, "W2 must be an FP8 tensor")
    _check(W2.is_contiguous(), "W2 must be contiguous")
    E = int(W2.size(0))
    _check(W2.size(1) == H and W2.size(2) == I_DIM, "W2 must be [E_local, 7168, 2048]")
    out = _check_out(out, (E, *W2_PACKED_SHAPE), W2, "pack_w2")
    if E == 0:
        return out
    with torch.cuda.device(W2.device):
        capi.check(capi.load().moe_pack_w2(_ptr(W2), _ptr(out), E, _stream(W2.device)), "pack_w2")
    return out


def unpack_w13(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_w13, returned as uint8 [E, 4096, 7168]."""
    _require_device("W13_packed", packed)
    _check(packed.dim() == 7 and tuple(packed.shape[1:]) == W13_PACKED_SHAPE and packed.is_contiguous(),
           "W13_packed must be [E_local, 16, 56, 16, 2, 64, 4] contiguous")
    E = int(packed.size(0))
    out = torch.empty((E, 2 * I_DIM, H), dtype=torch.uint8, device=packed.device)
    with torch.cuda.device(packed.device):
        capi.check(capi.load().moe_unpack_w13(_ptr(packed), _ptr(out), E, _stream(packed.device)), "unpack_w13")
    return out


def unpack_w2(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_w2, returned as uint8 [E, 7168, 2048]."""
    _require_device("W2_packed", packed)
    _check(packed.dim() == 7 and tuple(packed.shape[1:]) == W2_PACKED_SHAPE and packed.is_contiguous(),
           "W2_packed must be [E_local, 56, 16, 8, 2, 64, 4] contiguous")
    E = int(packed.size(0))
    out = torch.empty((E, H, I_DIM), dtype=torch.uint8, device=packed.device)
    with torch.cuda.device(packed.device):
        capi.check(capi.load().moe_unpack_w2(_ptr(packed), _ptr(out), E, _stream(packed.device)), "unpack_w2")
    return out


# --------------------------------------------------------------------------- upstream producer
ROUTER_PACKED_SHAPE = (56, 4, 16, 64, 8)  # [kb, ks, expert tile, lane, bf16]


def pack_router(router_w: torch.Tensor) -> torch.Tensor:
    """Router weight bf16 [256, 7168] -> packed bf16 MFMA operand fragments
    (ROUTER_PACKED_SHAPE), for router_quant."""
    _require_device("router_w", router_w)
    _check(router_w.dtype == torch.bfloat16, "router_w must be bfloat16")
    _check(tuple(router_w.shape) == (E_GLOBAL, H) and router_w.is_contiguous(),
           "router_w must be [256, 7168] contiguous")
    out = torch.empty(ROUTER_PACKED_SHAPE, dtype=torch.bfloat16, device=router_w.device)
    with torch.cuda.device(router_w.device):
        capi.check(capi.load().moe_pack_router(_ptr(router_w), _ptr(out), _stream(router_w.device)), "pack_router")
    return out


def unpack_router(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_router."""
    _require_device("router_packed", packed)
    _check(tuple(packed.shape) == ROUTER_PACKED_SHAPE and packed.is_contiguous() and packed.dtype == torch.bfloat16,
           "router_packed must be a pack_router result")
    out = torch.empty((E_GLOBAL, H), dtype=torch.bfloat16, device=packed.device)
    with torch.cuda.device(packed.device):
        capi.check(capi.load().moe_unpack_router(_ptr(packed), _ptr(out), _stream(packed.device)), "unpack_router")
    return out


def router_quant(hidden: torch.Tensor, router_packed: torch.Tensor):
    """bf16 hidden states [T, 7168] -> (routing_logits f32 [T, 256],
    hidden_states e4m3 [T, 7168], hidden_states_scale f32 [56, T]): the
    router GEMM and the dynamic FP8 quantisation in front of moe_forward,
    in one pass over the hidden states (moe_router_quant)."""
    _require_device("hidden", hidden)
    dev = hidden.device
    _check(hidden.dtype == torch.bfloat16, "hidden must be bfloat16")
    _check(hidden.dim() == 2 and hidden.size(1) == H and hidden.is_contiguous(), "hidden must be [T, 7168] contiguous")
    _require_device("router_packed", router_packed, dev)
    _check(tuple(router_packed.shape) == ROUTER_PACKED_SHAPE and router_packed.dtype == torch.bfloat16,
           "router_packed must be a pack_router result")
    T = int(hidden.size(0))
    _check(T <= capi.MAX_T, f"T must be <= {capi.MAX_T}")
    lib = capi.load()
    logits = torch.empty((T, E_GLOBAL), dtype=torch.float32, device=dev)
    hq = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=dev)
    hs = torch.empty((H_BLOCKS, T), dtype=torch.float32, device=dev)
    ws_bytes = int(lib.moe_router_workspace_bytes(T))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        capi.check(lib.moe_router_quant(_ptr(hidden), _ptr(router_packed), T, _ptr(ws), ws_bytes, _ptr(logits),
                                        _ptr(hq), _ptr(hs), _stream(dev)), "router_quant")
    return logits, hq, hs


# --------------------------------------------------------------------------- forward
def _validate_forward(hidden, hidden_scale, W13_packed, W13_scale, W2_packed, W2_scale, logits, bias):
    """The checks of kernels/moe.cu:759-817, for this build's packed layout."""
    _check(hidden.dim() == 2, "hidden must be [T, 7168]")
    _check(hidden_scale.dim() == 2, "hidden_scale must be [56, T]")
    _check(W13_packed.dim() == 7, "W13_packed must be [E_local, 16, 56, 16, 2, 64, 4]")
    _check(W13_scale.dim() == 3, "W13_scale must be [E_local, 32, 56]")
    _check(W2_packed.dim() == 7, "W2_packed must be [E_local, 56, 16, 8, 2, 64, 4]")
    _check(W2_scale.dim() == 3, "W2_scale must be [E_local, 56, 16]")
    _check(logits.dim() == 2, "logits must be [T, 256]")
    _check(hidden.element_size() == 1, "hidden must be an FP8 tensor")
    _check(hidden_scale.dtype == torch.float32, "hidden_scale must be float32")
    _check(W13_packed.dtype == torch.int32, "W13_packed must be int32-packed FP8 fragments")
    _check(W13_scale.dtype == torch.float32, "W13_scale must be float32")
    _check(W2_packed.dtype == torch.int32, "W2_packed must be int32-packed FP8 fragments")
    _check(W2_scale.dtype == torch.float32, "W2_scale must be float32")
    _check(logits.dtype == torch.float32, "logits must be float32")
    _check(bias.dtype == torch.float32, "bias must be float32")
    T, H_dim = int(hidden.size(0)), int(hidden.size(1))
    E = int(W13_packed.size(0))
    _check(H_dim == H, "hidden must have hidden dim 7168")
    _check(hidden_scale.size(0) == H_BLOCKS and hidden_scale.size(1) == T, "hidden_scale must be [56, T]")
    _check(logits.size(0) == T and logits.size(1) == E_GLOBAL, "logits must be [T, 256]")
    _check(bias.numel() == E_GLOBAL, "bias must have 256 elements")
    _check(tuple(W13_packed.shape[1:]) == W13_PACKED_SHAPE, "W13_packed must be [E_local, 16, 56, 16, 2, 64, 4]")
    _check(tuple(W13_scale.shape) == (E, G1_BLOCKS, H_BLOCKS), "W13_scale must be [E_local, 32, 56]")
    _check(W2_packed.size(0) == E and tuple(W2_packed.shape[1:]) == W2_PACKED_SHAPE,
           "W2_packed must be [E_local, 56, 16, 8, 2, 64, 4]")
    _check(tuple(W2_scale.shape) == (E, H_BLOCKS, I_BLOCKS), "W2_scale must be [E_local, 56, 16]")
    _check(1 <= E <= MAX_E_LOCAL, f"E_local must be in [1, {MAX_E_LOCAL}], got {E}")
    for name, t in (("hidden", hidden), ("hidden_scale", hidden_scale), ("W13_packed", W13_packed),
                    ("W13_scale", W13_scale), ("W2_packed", W2_packed), ("W2_scale", W2_scale),
                    ("logits", logits), ("bias", bias)):
        _check(t.is_contiguous(), f"{name} must be contiguous")
        _require_device(name, t, hidden.device)
    return T, E


def moe_forward_workspace(hidden, hidden_scale, W13_packed, W13_scale, W2_packed, W2_scale, logits, bias,
                          rsf: float, local_offset: int):
    """moe_forward that also returns its workspace tensor (for inspection)."""
    _require_device("hidden", hidden)
    T, E = _validate_forward(hidden, hidden_scale, W13_packed, W13_scale, W2_packed, W2_scale, logits, bias)
    lib = capi.load()
    dev = hidden.device
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ws_bytes = int(lib.moe_workspace_bytes(T, E))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    if T == 0:
        return out, ws
    with torch.cuda.device(dev):
        rc = lib.moe_forward(_ptr(hidden), _ptr(hidden_scale), _ptr(W13_packed), _ptr(W13_scale), _ptr(W2_packed),
                             _ptr(W2_scale), _ptr(logits), _ptr(bias), float(rsf), int(local_offset), T, E,
                             _ptr(ws), ws_bytes, _ptr(out), _stream(dev))
    capi.check(rc, "moe_forward")
    return out, ws


def moe_forward(hidden, hidden_scale, W13_packed, W13_scale, W2_packed, W2_scale, logits, bias, rsf: float,
                local_offset: int) -> torch.Tensor:
    """bf16 [T, 7168] MoE forward; argument order of kernels/moe.cu:744-754."""
    return moe_forward_workspace(hidden, hidden_scale, W13_packed, W13_scale, W2_packed, W2_scale, logits, bias,
                                 rsf, local_offset)[0]


# --------------------------------------------------------------------------- inspection
def workspace_views(ws: torch.Tensor, T: int, E: int) -> dict:
    """Typed views of the MOE_WS_* buffers inside a forward/route workspace.

    ``Y`` rows of routes whose ``route_token`` entry has bit 31 set (the
    token's only local route) are not written by the forward: GEMM2 writes
    that token's bf16 output row directly, so those Y rows hold stale data.
    """
    off = capi.workspace_offsets(T, E)
    R = T * min(TOP_K, E)

    def view(idx, dtype, shape):
        n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
        return ws[off[idx]:off[idx] + n].view(dtype).view(shape)

    return {
        "topk_ids": view(capi.WS_TOPK_IDS, torch.int32, (T, TOP_K)),
        "topk_w": view(capi.WS_TOPK_W, torch.float32, (T, TOP_K)),
        "counts": view(capi.WS_COUNTS, torch.int32, (E,)),
        "offsets": view(capi.WS_OFFSETS, torch.int32, (E + 1,)),
        "route_token": view(capi.WS_ROUTE_TOKEN, torch.int32, (R,)),
        "route_weight": view(capi.WS_ROUTE_WEIGHT, torch.float32, (R,)),
        "token_route": view(capi.WS_TOKEN_ROUTE, torch.int32, (T, TOP_K)),
        "Cq": view(capi.WS_CQ, torch.uint8, (R, I_DIM)),
        "Cs": view(capi.WS_CS, torch.float32, (R, I_BLOCKS)),
        "Y": view(capi.WS_Y, torch.float32, (R, H)),
    }


def route(logits: torch.Tensor, bias: torch.Tensor, rsf: float, local_offset: int, e_local: int = 32) -> dict:
    """Routing + local dispatch only; returns the dispatch buffers (cloned)."""
    _require_device("logits", logits)
    _check(logits.dim() == 2 and logits.size(1) == E_GLOBAL, "logits must be [T, 256]")
    _check(logits.dtype == torch.float32 and bias.dtype == torch.float32, "logits and bias must be float32")
    _check(bias.numel() == E_GLOBAL, "bias must have 256 elements")
    _check(logits.is_contiguous() and bias.is_contiguous(), "logits and bias must be contiguous")
    _require_device("bias", bias, logits.device)
    lib = capi.load()
    T = int(logits.size(0))
    dev = logits.device
    ws_bytes = int(lib.moe_workspace_bytes(T, e_local))
    _check(ws_bytes > 0 or T == 0, f"invalid e_local {e_local}")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.moe_route(_ptr(logits), _ptr(bias), float(rsf), int(local_offset), T, int(e_local), _ptr(ws),
                           ws_bytes, _stream(dev))
    capi.check(rc, "moe_route")
    views = workspace_views(ws, T, e_local)
    keep = ("topk_ids", "topk_w", "counts", "offsets", "route_token", "route_weight", "token_route")
    return {k: views[k].clone() for k in keep}


# --------------------------------------------------------------------------- synthesis
def fill_normal_e4m3_(t: torch.Tensor, seed: int, stream_id: int) -> torch.Tensor:
    """In-place device fill with the counter-based ~N(0,1) e4m3 sequence."""
    _require_device("t", t)
    _check(t.element_size() == 1 and t.is_contiguous(), "t must be a contiguous 1-byte tensor")
    with torch.cuda.device(t.device):
        capi.check(capi.load().moe_fill_normal_e4m3(_ptr(t), t.numel(), int(seed), int(stream_id), _stream(t.device)),
                   "moe_fill_normal_e4m3")
    return t


def host_normal_e4m3(n: int, seed: int, stream_id: int, first_index: int = 0, threads: int = 0) -> np.ndarray:
    """Elements [first_index, first_index+n) of the same sequence, on the CPU."""
    out = np.empty(n, dtype=np.uint8)
    if n:
        rc = capi.load().moe_host_fill_normal_e4m3(out.ctypes.data_as(ctypes.c_void_p), n, int(seed), int(stream_id),
                                                   int(first_index), int(threads))
        capi.check(rc, "moe_host_fill_normal_e4m3")
    return out
