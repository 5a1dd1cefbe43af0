"""No-aux-loss DeepSeek-V3 routing restated in numpy (reference/moe_ref.py:81-107).

Steps (all fp32 unless noted):
  s  = sigmoid(logits)                              moe_ref.py:85
  v  = s + bias                                     moe_ref.py:86
  group score = sum of the two largest v per group  moe_ref.py:88-92
  keep the 4 best groups                            moe_ref.py:94-97
  top-8 experts by v over the kept groups           moe_ref.py:99-101
  w_k = s_k / (sum_k s_k + 1e-20) * rsf             moe_ref.py:103-107

Tie convention (the reference's torch.topk leaves it unspecified): larger
value first, then the lower index -- the choice of the reference kernel
(kernels/moe.cu:153,294).  The 8 weights are summed in ascending expert
order; that fixes the fp32 rounding of the denominator.
"""

from __future__ import annotations

import numpy as np

from .numerics import sigmoid

E_GLOBAL, N_GROUP, GROUP_SIZE, TOP_K, TOPK_GROUP = 256, 8, 32, 8, 4


def route(logits: np.ndarray, bias: np.ndarray, rsf: float) -> dict:
    """Returns ids [T,8] (ascending global expert), weights [T,8] fp32,
    group_mask [T,8] bool, and decision margins for diagnosis."""
    logits = np.asarray(logits, dtype=np.float32)
    bias = np.asarray(bias, dtype=np.float32).reshape(-1)
    T = logits.shape[0]
    s = sigmoid(logits)
    v = (s + bias[None, :]).astype(np.float32)

    grouped = v.reshape(T, N_GROUP, GROUP_SIZE)
    top2 = np.sort(grouped, axis=2)[:, :, -2:]
    gscore = (top2[:, :, 1] + top2[:, :, 0]).astype(np.float32)
    gorder = np.argsort(-gscore, axis=1, kind="stable")
    group_mask = np.zeros((T, N_GROUP), dtype=bool)
    np.put_along_axis(group_mask, gorder[:, :TOPK_GROUP], True, axis=1)

    cand = np.where(np.repeat(group_mask, GROUP_SIZE, axis=1), v, np.float32(-np.inf))
    order = np.argsort(-cand, axis=1, kind="stable")
    ids = np.sort(order[:, :TOP_K], axis=1).astype(np.int32)

    sw = np.take_along_axis(s, ids, axis=1)
    total = sw[:, 0].copy()
    for k in range(1, TOP_K):
        total = (total + sw[:, k]).astype(np.float32)
    total = (total + np.float32(1e-20)).astype(np.float32)
    w = ((sw / total[:, None]).astype(np.float32) * np.float32(rsf)).astype(np.float32)

    rows = np.arange(T)[:, None]
    sorted_cand = np.take_along_axis(cand, order[:, : TOP_K + 1], axis=1)
    gs_sorted = np.take_along_axis(gscore, gorder, axis=1)
    return {
        "ids": ids,
        "weights": w,
        "group_mask": group_mask,
        "expert_margin": (sorted_cand[:, TOP_K - 1] - sorted_cand[:, TOP_K]).astype(np.float64),
        "group_margin": (gs_sorted[:, TOPK_GROUP - 1] - gs_sorted[:, TOPK_GROUP]).astype(np.float64),
        "_rows": rows,
    }


def route_bruteforce(logits: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """Top-8 sets by exhaustive search over the C(8,4) group choices: the kept
    groups are the choice with the largest multiset of group scores; the
    experts are the 8 best of the kept 128.  Pure Python, small T only."""
    from itertools import combinations

    logits = np.asarray(logits, dtype=np.float32)
    bias = np.asarray(bias, dtype=np.float32)
    v = (sigmoid(logits) + bias[None, :]).astype(np.float32)
    out = []
    for t in range(v.shape[0]):
        gs = []
        for g in range(N_GROUP):
            vals = sorted(v[t, g * GROUP_SIZE:(g + 1) * GROUP_SIZE].tolist(), reverse=True)
            gs.append(float(np.float32(vals[0]) + np.float32(vals[1])))
        best, best_key = None, None
        for combo in combinations(range(N_GROUP), TOPK_GROUP):
            # the 4 kept scores, compared as a sorted vector; ties -> lower indices
            key = (sorted((gs[g] for g in combo), reverse=True), [-g for g in combo])
            if best_key is None or key > best_key:
                best, best_key = combo, key
        cands = [(float(v[t, e]), -e) for g in best for e in range(g * GROUP_SIZE, (g + 1) * GROUP_SIZE)]
        cands.sort(reverse=True)
        out.append(sorted(-c[1] for c in cands[:TOP_K]))
    return np.asarray(out, dtype=np.int32)


# route_token entries of routes whose token has no other local route carry
# this bit (the GEMM2 kernels write those tokens' output rows themselves).
SINGLE_ROUTE_FLAG = np.int32(-(2 ** 31))


def local_dispatch(ids: np.ndarray, weights: np.ndarray, local_offset: int, e_local: int) -> dict:
    """Token-ordered per-expert route lists (the dispatch the GPU builds):
    route r of local expert e sits at offsets[e] + (rank of its token among
    the expert's tokens); route_token[r] is the token, with bit 31
    (SINGLE_ROUTE_FLAG) set when that token has exactly one local route."""
    T = ids.shape[0]
    le = ids - int(local_offset)
    local = (le >= 0) & (le < e_local)
    counts = np.array([int(np.count_nonzero(local & (le == e))) for e in range(e_local)], dtype=np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = int(offsets[-1])
    route_token = np.full(R, -1, np.int32)
    route_weight = np.zeros(R, np.float32)
    token_route = np.full((T, TOP_K), -1, np.int32)
    fill = offsets[:-1].copy()
    n_local = local.sum(axis=1)
    for t in range(T):
        j = 0
        for k in range(TOP_K):  # ids ascending -> local experts ascending
            if local[t, k]:
                e = le[t, k]
                r = fill[e]
                fill[e] += 1
                # bit 31 flags the route of a token with a single local route
                route_token[r] = t | (SINGLE_ROUTE_FLAG if n_local[t] == 1 else 0)
                route_weight[r] = weights[t, k]
                token_route[t, j] = r
                j += 1
    return {"counts": counts, "offsets": offsets, "route_token": route_token, "route_weight": route_weight,
            "token_route": token_route}
