"""Host-side logic that needs no GPU: the ops surface refuses CPU tensors
(no CPU path), shape/dtype validation mirrors kernels/moe.cu:705-817, the
packed-weight cache semantics of moe_layer.py:77-95, and the synthetic
input configs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import pkg


def test_ops_refuse_cpu_tensors(ops):
    w13 = torch.zeros((1, 4096, 7168), dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ops.pack_w13(w13)
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ops.pack_w2(torch.zeros((1, 7168, 2048), dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ops.moe_forward(*[torch.zeros(1)] * 8, 1.0, 0)
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ops.route(torch.zeros((2, 256)), torch.zeros(256), 1.0, 0)


def _valid_meta(T=4, E=2):
    f8, f32, i32 = torch.float8_e4m3fn, torch.float32, torch.int32
    return dict(
        hidden=torch.zeros((T, 7168), dtype=f8),
        hidden_scale=torch.zeros((56, T), dtype=f32),
        W13_packed=torch.zeros((E, 16, 56, 16, 2, 64, 4), dtype=i32),
        W13_scale=torch.zeros((E, 32, 56), dtype=f32),
        W2_packed=torch.zeros((E, 56, 16, 8, 2, 64, 4), dtype=i32),
        W2_scale=torch.zeros((E, 56, 16), dtype=f32),
        logits=torch.zeros((T, 256), dtype=f32),
        bias=torch.zeros(256, dtype=f32),
    )


@pytest.mark.parametrize("key,bad,msg", [
    ("hidden", torch.zeros((4, 7168, 1), dtype=torch.uint8), r"hidden must be \[T, 7168\]"),
    ("hidden", torch.zeros((4, 7168), dtype=torch.float16), "hidden must be an FP8 tensor"),
    ("hidden", torch.zeros((4, 7000), dtype=torch.uint8), "hidden must have hidden dim 7168"),
    ("hidden_scale", torch.zeros((4, 56)), r"hidden_scale must be \[56, T\]"),
    ("hidden_scale", torch.zeros((56, 4), dtype=torch.float16), "hidden_scale must be float32"),
    ("W13_packed", torch.zeros((2, 16, 56, 16, 2, 64, 4), dtype=torch.int64), "W13_packed must be int32"),
    ("W13_scale", torch.zeros((2, 32, 55)), r"W13_scale must be \[E_local, 32, 56\]"),
    ("W2_packed", torch.zeros((3, 56, 16, 8, 2, 64, 4), dtype=torch.int32), r"W2_packed must be"),
    ("W2_scale", torch.zeros((2, 56, 15)), r"W2_scale must be \[E_local, 56, 16\]"),
    ("logits", torch.zeros((4, 255)), r"logits must be \[T, 256\]"),
    ("logits", torch.zeros((5, 256)), r"logits must be \[T, 256\]"),
    ("bias", torch.zeros(255), "bias must have 256 elements"),
    ("bias", torch.zeros(256, dtype=torch.bfloat16), "bias must be float32"),
    ("hidden", torch.zeros((7168, 4), dtype=torch.uint8).t(), "hidden must be contiguous"),
])
def test_forward_validation(ops, key, bad, msg):
    args = _valid_meta()
    args[key] = bad
    with pytest.raises(RuntimeError, match=msg):
        ops._validate_forward(**args)


def test_forward_validation_e_local_limit(ops):
    args = _valid_meta(E=33)
    with pytest.raises(RuntimeError, match="E_local must be in"):
        ops._validate_forward(**args)


def test_forward_validation_reaches_device_check(ops):
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ops._validate_forward(**_valid_meta())


def test_cached_pack_semantics():
    layer = pkg("moe_layer")
    calls = []

    def fake_pack(t):
        calls.append(t)
        return t.clone()

    layer._packed_weight_cache.clear()
    w = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    a = layer._cached_pack("w13", w, fake_pack)
    b = layer._cached_pack("w13", w, fake_pack)
    assert a is b and len(calls) == 1
    layer._cached_pack("w2", w, fake_pack)
    assert len(calls) == 2                     # different name
    w.add_(1)                                  # in-place update bumps _version
    c = layer._cached_pack("w13", w, fake_pack)
    assert len(calls) == 3 and torch.equal(c, w)
    other = w.clone()
    layer._cached_pack("w13", other, fake_pack)
    assert len(calls) == 4                     # different storage
    layer._packed_weight_cache.clear()


def test_load_custom_ops_surface():
    layer = pkg("moe_layer")
    ops = layer._load_custom_ops()
    for name in ("pack_w13", "pack_w2", "moe_forward"):
        assert callable(getattr(ops, name))
    assert layer._load_custom_ops() is ops


def test_config_table(inputs_mod):
    assert [c.T for c in inputs_mod.CONFIGS.values()] == [16, 64, 1024, 8192, 4096]
    assert inputs_mod.CONFIGS[2].local_expert_offset == 96
    assert inputs_mod.CONFIGS[4].skewed
    assert all(c.rsf == 2.5 for c in inputs_mod.CONFIGS.values())


def test_config_small_tensors(inputs_mod):
    cfg = inputs_mod.CONFIGS[1]
    a = inputs_mod.host_tensors(cfg)
    b = inputs_mod.host_tensors(cfg)
    for k in a:
        assert torch.equal(a[k], b[k]), k
    assert a["routing_bias"].dtype == torch.bfloat16
    assert a["hidden_states_scale"].shape == (56, 64)
    hs = a["hidden_states_scale"]
    assert float(hs.min()) >= 0.01 and float(hs.max()) <= 0.05
    ws = a["gemm1_weights_scale"]
    assert ws.shape == (32, 32, 56) and float(ws.min()) >= 0.001 and float(ws.max()) <= 0.01
    lg = a["routing_logits"]
    assert abs(float(lg.mean())) < 0.02 and abs(float(lg.std()) - 1.0) < 0.02
    bias = a["routing_bias"].float()
    assert 0.05 < float(bias.std()) < 0.15
    skew = inputs_mod.host_tensors(inputs_mod.CONFIGS[4])["routing_bias"].float()
    assert skew[:4].tolist() == [3.0] * 4 and float(skew[4:].abs().max()) == 0.0


def test_config_inputs_cpu_shapes(inputs_mod):
    inp = inputs_mod.make_config_inputs(0, device="cpu")
    assert list(inp) == ["routing_logits", "routing_bias", "hidden_states", "hidden_states_scale", "gemm1_weights",
                         "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale", "local_expert_offset",
                         "routed_scaling_factor"]
    assert inp["hidden_states"].dtype == torch.float8_e4m3fn and inp["hidden_states"].shape == (16, 7168)
    assert inp["gemm1_weights"].shape == (32, 4096, 7168)
    assert inp["gemm2_weights"].shape == (32, 7168, 2048)
    sample = inp["gemm1_weights"][3, :64].float()
    assert abs(float(sample.mean())) < 0.01 and abs(float(sample.std()) - 1.0) < 0.02
    w13, w2 = inputs_mod.expert_weights_host(inputs_mod.CONFIGS[0], [3, 17])
    assert np.array_equal(w13[0], inp["gemm1_weights"][3].view(torch.uint8).numpy())
    assert np.array_equal(w2[1], inp["gemm2_weights"][17].view(torch.uint8).numpy())


def test_geometry_matches_kernel_constants():
    """The host constants bench.py and the tests use agree with the kernels'."""
    import re
    from pathlib import Path

    geo = pkg("geometry")
    common = (Path(__file__).resolve().parents[1] / "15642_moe_amd" / "csrc" / "common.h").read_text()
    for name, value in (("DECODE_MAX_T", geo.DECODE_MAX_T), ("MAX_E_LOCAL", geo.MAX_E_LOCAL)):
        m = re.search(rf"constexpr int {name} = (\d+);", common)
        assert m and int(m.group(1)) == value, name


@pytest.mark.parametrize("seed", range(40))
def test_item_queue_protocol_claims_every_item_once(seed):
    """The prefill GEMMs' work distribution (gemm_util.h ItemQueue), played
    as its atomics under random interleavings of the workgroups: per-XCD
    claim counters over nq contiguous segments, a workgroup stealing from
    the next undrained segment once its own is drained, and a drained-mask
    word whose atomicOr result lets it skip segments others found drained.
    Every item must be taken exactly once, and each workgroup must stop
    after at most nq claims beyond the items it takes."""
    rng = np.random.default_rng(seed)
    nq = int(rng.integers(1, 9))
    n_work = int(rng.choice([0, 1, 5, nq, 37, 256, 1000]))
    n_wg = int(rng.integers(1, 64))
    counters = [0] * nq
    mask = 0
    seg = [n_work * x // nq for x in range(nq + 1)]

    def workgroup(q):
        nonlocal mask
        cur, claims = q % nq, 0

        def claim():
            nonlocal claims
            claims += 1
            c = counters[cur]
            counters[cur] += 1
            return c
        claimed = claim()
        yield None  # the atomic's round trip: other workgroups run here
        while True:
            L = seg[cur] + claimed
            if L < seg[cur + 1]:
                yield ("item", L, claims)
                claimed = claim()
                yield None
                continue
            old = mask
            mask |= 1 << cur
            m = old | (1 << cur)
            yield None
            if m & ((1 << nq) - 1) == (1 << nq) - 1:
                yield ("done", None, claims)
                return
            cur = (cur + 1) % nq
            while (m >> cur) & 1:
                cur = (cur + 1) % nq
            claimed = claim()
            yield None

    live = {p: workgroup(p) for p in range(n_wg)}
    taken, items_of = [], {p: 0 for p in range(n_wg)}
    while live:
        p = list(live)[int(rng.integers(len(live)))]
        ev = next(live[p])
        if ev is None:
            continue
        kind, L, claims = ev
        if kind == "item":
            taken.append(L)
            items_of[p] += 1
        else:
            assert claims <= items_of[p] + nq + 1
            del live[p]
    assert sorted(taken) == list(range(n_work))
