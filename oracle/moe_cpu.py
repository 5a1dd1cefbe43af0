"""CPU models of the MoE forward (torch on the CPU).

forward_reference   the semantics of reference/moe_ref.py:5-136 in fp32:
                    block dequant (:58-79), routing (:81-107), per local
                    expert GEMM1 -> SwiGLU (silu on rows I..2I-1) -> GEMM2
                    (:113-131), weighted index_add in local-expert order
                    (:134), bf16 (:136).  Dequantises only the experts that
                    receive routes (same per-element arithmetic as a full
                    dequant).  `routing="torch"` uses the reference's own op
                    sequence (torch.sigmoid / torch.topk); `routing="oracle"`
                    uses oracle.routing (the GPU's sigmoid evaluation).
forward_full_dequant the same with the reference's full up-front dequant of
                    all 32 experts -- the timed CPU baseline.
kernel_model        the FP8 kernel's numerics: exact per-128-K block sums
                    rounded to fp32, x (act_scale * w_scale) accumulated in
                    fp32 (kernels/moe.cu:468-493, 652-667), SwiGLU, C requant
                    to e4m3 with scale max(amax/448, 1e-8) (:516-541), GEMM2
                    likewise, y = O * w, per-token sum in ascending expert
                    order, bf16 RNE.
"""

from __future__ import annotations

import numpy as np
import torch

from . import routing as oracle_routing
from .numerics import E4M3_TABLE, bf16_bits, e4m3_encode

H, I, E_GLOBAL, BLOCK = 7168, 2048, 256, 128
N_GROUP, TOP_K, TOPK_GROUP = 8, 8, 4


def _u8(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().contiguous().view(torch.uint8).numpy()
    return np.asarray(t, dtype=np.uint8)


def _f32(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().to(torch.float32).contiguous().numpy()
    return np.asarray(t, dtype=np.float32)


def _fp8_to_f32(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(E4M3_TABLE[b].astype(np.float32))


# --------------------------------------------------------------------------- routing
def route_torch(logits: torch.Tensor, bias: torch.Tensor, rsf: float):
    """The reference's routing op sequence (moe_ref.py:81-107) on CPU tensors.
    Returns (topk_idx [T,8] int64, unsorted; dense weights [T,256] fp32)."""
    logits = logits.to(torch.float32)
    bias = bias.to(torch.float32).reshape(-1)
    T = logits.shape[0]
    s = torch.sigmoid(logits)
    s_wb = s + bias
    grouped = s_wb.view(T, N_GROUP, E_GLOBAL // N_GROUP)
    top2, _ = torch.topk(grouped, k=2, dim=2, largest=True, sorted=False)
    gscore = top2.sum(dim=2)
    _, gidx = torch.topk(gscore, k=TOPK_GROUP, dim=1, largest=True, sorted=False)
    gmask = torch.zeros_like(gscore)
    gmask.scatter_(1, gidx, 1.0)
    smask = gmask.unsqueeze(2).expand(T, N_GROUP, E_GLOBAL // N_GROUP).reshape(T, E_GLOBAL)
    pruned = s_wb.masked_fill(smask == 0, torch.finfo(torch.float32).min)
    _, topk_idx = torch.topk(pruned, k=TOP_K, dim=1, largest=True, sorted=False)
    M = torch.zeros_like(s)
    M.scatter_(1, topk_idx, 1.0)
    w = s * M
    w = (w / (w.sum(dim=1, keepdim=True) + 1e-20)) * rsf
    return topk_idx, w


def _routing(inputs: dict, routing: str):
    logits, bias = inputs["routing_logits"].cpu(), inputs["routing_bias"].cpu()
    rsf = float(inputs["routed_scaling_factor"])
    if routing == "torch":
        idx, dense = route_torch(logits, bias, rsf)
        ids = torch.sort(idx, dim=1).values
        return ids.numpy().astype(np.int32), torch.gather(dense, 1, ids).numpy()
    r = oracle_routing.route(_f32(logits), _f32(bias), rsf)
    return r["ids"], r["weights"]


# --------------------------------------------------------------------------- reference semantics
def forward_reference(inputs: dict, routing: str = "oracle", ids=None, weights=None,
                      token_subset=None) -> torch.Tensor:
    """fp32 reference semantics -> bf16 [T, H] (rows outside `token_subset`,
    when given, are left zero).  `ids`/`weights` override the routing."""
    if ids is None:
        ids, weights = _routing(inputs, routing)
    T = ids.shape[0]
    offset = int(inputs["local_expert_offset"])
    E = int(inputs["gemm1_weights"].shape[0])
    tokens = np.arange(T) if token_subset is None else np.asarray(sorted(token_subset))
    a_bytes = _u8(inputs["hidden_states"])
    a_scale = _f32(inputs["hidden_states_scale"])          # [56, T]
    w13 = inputs["gemm1_weights"]
    w2 = inputs["gemm2_weights"]
    s13 = torch.from_numpy(_f32(inputs["gemm1_weights_scale"]))
    s2 = torch.from_numpy(_f32(inputs["gemm2_weights_scale"]))
    out = torch.zeros((T, H), dtype=torch.float32)
    for le in range(E):
        ge = offset + le
        if ge < 0 or ge >= E_GLOBAL:
            continue
        hit = (ids[tokens] == ge).any(axis=1)
        if not hit.any():
            continue
        tok = tokens[hit]
        A = _fp8_to_f32(a_bytes[tok]) * torch.from_numpy(np.repeat(a_scale[:, tok].T, BLOCK, axis=1))
        W13 = _fp8_to_f32(_u8(w13[le])) * torch.repeat_interleave(torch.repeat_interleave(s13[le], BLOCK, 0), BLOCK, 1)
        W2 = _fp8_to_f32(_u8(w2[le])) * torch.repeat_interleave(torch.repeat_interleave(s2[le], BLOCK, 0), BLOCK, 1)
        G1 = A.matmul(W13.t())
        X1, X2 = G1[:, :I], G1[:, I:]
        C = (X2 / (1.0 + torch.exp(-X2))) * X1
        O = C.matmul(W2.t())
        k = np.argmax(ids[tok] == ge, axis=1)
        wt = torch.from_numpy(np.asarray(weights)[tok, k].astype(np.float32))
        out.index_add_(0, torch.from_numpy(tok), O * wt.unsqueeze(1))
    return out.to(torch.bfloat16)


def forward_full_dequant(inputs: dict) -> torch.Tensor:
    """moe_ref.py's algorithm with its full up-front dequantisation (timed as
    the CPU baseline): inputs are CPU tensors."""
    T = inputs["routing_logits"].shape[0]
    A = inputs["hidden_states"].to(torch.float32) * inputs["hidden_states_scale"].to(torch.float32).t() \
        .repeat_interleave(BLOCK, dim=1)
    S13 = inputs["gemm1_weights_scale"].to(torch.float32)
    W13 = inputs["gemm1_weights"].to(torch.float32) * S13.repeat_interleave(BLOCK, 1).repeat_interleave(BLOCK, 2)
    S2 = inputs["gemm2_weights_scale"].to(torch.float32)
    W2 = inputs["gemm2_weights"].to(torch.float32) * S2.repeat_interleave(BLOCK, 1).repeat_interleave(BLOCK, 2)
    idx, dense = route_torch(inputs["routing_logits"], inputs["routing_bias"], float(inputs["routed_scaling_factor"]))
    out = torch.zeros((T, H), dtype=torch.float32)
    offset = int(inputs["local_expert_offset"])
    for le in range(W13.shape[0]):
        ge = offset + le
        if ge < 0 or ge >= E_GLOBAL:
            continue
        sel = (idx == ge).any(dim=1)
        if not sel.any():
            continue
        tok = torch.nonzero(sel, as_tuple=False).squeeze(1)
        G1 = A.index_select(0, tok).matmul(W13[le].t())
        X1, X2 = G1[:, :I], G1[:, I:]
        C = (X2 / (1.0 + torch.exp(-X2))) * X1
        O = C.matmul(W2[le].t())
        out.index_add_(0, tok, O * dense.index_select(0, tok)[:, ge].unsqueeze(1))
    return out.to(torch.bfloat16)


# --------------------------------------------------------------------------- kernel semantics
def _fma32(a, b, c):
    """fp32 fused multiply-add (exact product and sum in float64, one final
    rounding; double rounding through float64 is ignored).  Accepts numpy
    arrays or torch tensors (torch runs the elementwise work on all host
    threads); returns the same kind as `a`."""
    if isinstance(a, np.ndarray):
        return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)
    return (a.double() * b.double() + c.double()).float()


def weight_operand(w: np.ndarray, nblk: int) -> torch.Tensor:
    """e4m3 weight bytes [N, nblk*128] -> float64 [nblk, 128, N] (the right
    operand of _block_sums; prepare once per expert and reuse)."""
    return torch.from_numpy(E4M3_TABLE[w].reshape(w.shape[0], nblk, BLOCK)).permute(1, 2, 0).contiguous()


def _block_sums(a: np.ndarray, w: np.ndarray, nblk: int, w_op: torch.Tensor | None = None) -> torch.Tensor:
    """Exact per-128-K block dot products rounded to fp32 (float64 sums of
    e4m3 x e4m3 products are exact: each product has 8 significant bits
    within 2^-18 .. 2^18, so 128 of them fit the 53-bit significand).
    a: [R, nblk*128] bytes, w: [N, nblk*128] bytes (or w_op, its
    weight_operand) -> [nblk, R, N] fp32."""
    A = torch.from_numpy(E4M3_TABLE[a].reshape(a.shape[0], nblk, BLOCK)).permute(1, 0, 2)
    W = weight_operand(w, nblk) if w_op is None else w_op
    return torch.bmm(A, W).to(torch.float32)


def _scaled_accumulate(raw: torch.Tensor, a_scale: np.ndarray, w_scale_rows: np.ndarray) -> np.ndarray:
    """acc = fma(raw[kb], a_scale[:, kb] * w_scale_rows[:, kb], acc) over the
    K-blocks in order, in fp32 (kernels/moe.cu:468-493, 652-667)."""
    a_s = torch.from_numpy(np.ascontiguousarray(a_scale, dtype=np.float32))
    w_s = torch.from_numpy(np.ascontiguousarray(w_scale_rows, dtype=np.float32))
    acc = torch.zeros(raw.shape[1:], dtype=torch.float32)
    for kb in range(raw.shape[0]):
        sc = a_s[:, kb][:, None] * w_s[:, kb][None, :]  # fp32 product, as the kernel forms it
        acc = _fma32(raw[kb], sc, acc)
    return acc.numpy()


def stage1_model(a_bytes, a_scale, w13_bytes, w13_scale, w_op=None):
    """One expert.  a_bytes [R,7168] u8, a_scale [R,56] f32, w13_bytes
    [4096,7168] u8, w13_scale [32,56] f32 -> (Cq [R,2048] u8, Cs [R,16] f32,
    c [R,2048] f32 before requant)."""
    raw = _block_sums(a_bytes, w13_bytes, H // BLOCK, w_op)            # [56, R, 4096]
    wsc = np.repeat(np.asarray(w13_scale, np.float32), BLOCK, axis=0)  # [4096, 56]
    acc = _scaled_accumulate(raw, a_scale, wsc)
    gate = torch.from_numpy(acc[:, :I])
    up = torch.from_numpy(acc[:, I:])
    c = ((up / (1.0 + torch.exp(-up))) * gate).numpy()
    R = c.shape[0]
    amax = np.abs(c.reshape(R, I // BLOCK, BLOCK)).max(axis=2)
    scale = np.maximum((amax / np.float32(448.0)).astype(np.float32), np.float32(1e-8)).astype(np.float32)
    q = (c.reshape(R, I // BLOCK, BLOCK) / scale[:, :, None]).astype(np.float32)
    q = np.clip(q, np.float32(-448.0), np.float32(448.0))
    return e4m3_encode(q.reshape(R, I)), scale, c


def stage2_model(cq, cs, w2_bytes, w2_scale, w_op=None):
    """One expert.  cq [R,2048] u8, cs [R,16] f32, w2_bytes [7168,2048] u8,
    w2_scale [56,16] f32 -> O [R,7168] f32."""
    raw = _block_sums(cq, w2_bytes, I // BLOCK, w_op)                  # [16, R, 7168]
    wsc = np.repeat(np.asarray(w2_scale, np.float32), BLOCK, axis=0)   # [7168, 16]
    return _scaled_accumulate(raw, cs, wsc)


def kernel_model(inputs: dict, ids=None, weights=None, token_subset=None, keep_intermediates: bool = False,
                 route_chunk: int = 512, progress=None):
    """FP8-kernel semantics -> dict(out_bf16_bits [T,H] uint16, and per-expert
    intermediates keyed by local expert when `keep_intermediates`).

    Each expert's routes are modelled `route_chunk` at a time (every route is
    independent through both GEMMs), which bounds host memory at any T; the
    per-token sums run in ascending local-expert order, fp32, starting from
    0 + y (the kernel's combine order).  `progress(local_expert, n_routes)`,
    when given, is called after each expert."""
    if ids is None:
        r = oracle_routing.route(_f32(inputs["routing_logits"]), _f32(inputs["routing_bias"]),
                                 float(inputs["routed_scaling_factor"]))
        ids, weights = r["ids"], r["weights"]
    T = ids.shape[0]
    offset = int(inputs["local_expert_offset"])
    E = int(inputs["gemm1_weights"].shape[0])
    tokens = np.arange(T) if token_subset is None else np.asarray(sorted(token_subset))
    a_bytes = _u8(inputs["hidden_states"])
    a_scale = _f32(inputs["hidden_states_scale"])
    s13 = _f32(inputs["gemm1_weights_scale"])
    s2 = _f32(inputs["gemm2_weights_scale"])
    out = np.zeros((T, H), dtype=np.float32)
    inter = {}
    for le in range(E):
        ge = offset + le
        hit = (ids[tokens] == ge).any(axis=1)
        if not hit.any():
            continue
        tok_all = tokens[hit]
        w13b, w2b = _u8(inputs["gemm1_weights"][le]), _u8(inputs["gemm2_weights"][le])
        w13_op, w2_op = weight_operand(w13b, H // BLOCK), weight_operand(w2b, I // BLOCK)
        parts = []
        for c0 in range(0, len(tok_all), route_chunk):
            tok = tok_all[c0:c0 + route_chunk]
            cq, cs, c = stage1_model(a_bytes[tok], a_scale[:, tok].T.copy(), w13b, s13[le], w13_op)
            O = stage2_model(cq, cs, w2b, s2[le], w2_op)
            k = np.argmax(ids[tok] == ge, axis=1)
            wt = np.asarray(weights)[tok, k].astype(np.float32)
            Y = (O * wt[:, None]).astype(np.float32)
            out[tok] = (out[tok] + Y).astype(np.float32)  # a token appears once per expert
            if keep_intermediates:
                parts.append(dict(tokens=tok, Cq=cq, Cs=cs, c=c, O=O, Y=Y))
        if keep_intermediates:
            inter[le] = {key: np.concatenate([pt[key] for pt in parts]) for key in parts[0]}
        if progress is not None:
            progress(le, len(tok_all))
    res = {"out_bits": bf16_bits(out), "ids": ids, "weights": weights}
    if keep_intermediates:
        res["experts"] = inter
    return res
