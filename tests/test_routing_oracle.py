"""The routing oracle pinned against the reference's own routing op sequence
(golden fixtures at all five configs), brute force, known answers and
invariants."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import moe_cpu, routing
from oracle.numerics import sigmoid


def _cfg_routing(inputs_mod, idx):
    cfg = inputs_mod.CONFIGS[idx]
    small = inputs_mod.host_tensors(cfg)
    return cfg, small["routing_logits"], small["routing_bias"]


@pytest.mark.parametrize("idx", [0, 1, 2, 3, 4])
def test_oracle_matches_golden_reference_routing(inputs_mod, idx):
    cfg, logits, bias = _cfg_routing(inputs_mod, idx)
    fx = np.load(GOLDEN / f"routing_cfg{idx}.npz")
    assert str(fx["logits_sha256"]) == inputs_mod.sha256(logits), "input generator drifted"
    assert str(fx["bias_sha256"]) == inputs_mod.sha256(bias)
    r = routing.route(logits.numpy(), bias.to(torch.float32).numpy(), cfg.rsf)
    assert np.array_equal(r["ids"], fx["ids"])
    rel = np.abs(r["weights"] - fx["weights"]) / np.abs(fx["weights"])
    assert rel.max() < 1e-6  # the fixture sums the weights in torch's order


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("skew", [False, True])
def test_oracle_matches_bruteforce(seed, skew):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((48, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    if skew:
        bias[:] = 0
        bias[rng.choice(256, 6, replace=False)] = 3.0
    r = routing.route(logits, bias, 2.5)
    assert np.array_equal(r["ids"], routing.route_bruteforce(logits, bias))


def test_oracle_matches_torch_sequence_on_random_inputs():
    rng = np.random.default_rng(7)
    logits = torch.from_numpy(rng.standard_normal((2048, 256)).astype(np.float32))
    bias = torch.from_numpy((rng.standard_normal(256) * 0.1).astype(np.float32)).to(torch.bfloat16)
    idx, _ = moe_cpu.route_torch(logits, bias, 1.0)
    r = routing.route(logits.numpy(), bias.to(torch.float32).numpy(), 1.0)
    assert np.array_equal(torch.sort(idx, 1).values.numpy(), r["ids"])


def test_known_answer_single_group():
    # group 5 holds the 8 largest logits and the best group score -> picks 160..167
    logits = np.full((1, 256), -4.0, dtype=np.float32)
    logits[0, 160:168] = np.linspace(4.0, 3.0, 8)
    r = routing.route(logits, np.zeros(256, np.float32), 1.0)
    assert r["ids"][0].tolist() == list(range(160, 168))
    assert r["group_mask"][0, 5]


def test_known_answer_group_filter_beats_raw_score():
    # expert 255 alone has the best score, but its group's top-2 sum is the
    # worst of the 8, so it is never eligible.
    logits = np.zeros((1, 256), dtype=np.float32)
    for g in range(7):
        logits[0, g * 32:(g * 32) + 2] = 2.0 - 0.1 * g
    logits[0, 255] = 6.0
    logits[0, 224:255] = -8.0
    r = routing.route(logits, np.zeros(256, np.float32), 1.0)
    assert 255 not in r["ids"][0]
    assert not r["group_mask"][0, 7]
    assert r["group_mask"][0, :4].all()


def test_known_answer_bias_selects_but_does_not_weight():
    # +3 bias on experts 0..3 forces them in; weights use the unbiased sigmoid
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((16, 256)).astype(np.float32)
    bias = np.zeros(256, np.float32)
    bias[:4] = 3.0
    r = routing.route(logits, bias, 2.5)
    assert (r["ids"][:, :4] == np.arange(4)).all()
    s = sigmoid(logits)
    picked = np.take_along_axis(s, r["ids"], 1)
    np.testing.assert_allclose(r["weights"], picked / picked.sum(1, keepdims=True) * 2.5, rtol=1e-6)


def test_ties_prefer_lower_index():
    logits = np.zeros((1, 256), dtype=np.float32)  # all equal
    r = routing.route(logits, np.zeros(256, np.float32), 1.0)
    assert r["ids"][0].tolist() == list(range(8))  # group 0, experts 0..7
    assert r["group_mask"][0].tolist() == [True] * 4 + [False] * 4
    np.testing.assert_array_equal(r["weights"][0], np.full(8, np.float32(0.125)))


@pytest.mark.parametrize("idx", [1, 4])
def test_weight_invariants(inputs_mod, idx):
    cfg, logits, bias = _cfg_routing(inputs_mod, idx)
    r = routing.route(logits.numpy(), bias.to(torch.float32).numpy(), cfg.rsf)
    np.testing.assert_allclose(r["weights"].astype(np.float64).sum(1), cfg.rsf, rtol=2e-6)
    assert (np.diff(r["ids"], axis=1) > 0).all()
    groups = r["ids"] // 32
    for t in range(groups.shape[0]):
        assert set(groups[t]) <= set(np.nonzero(r["group_mask"][t])[0])
    assert (r["group_mask"].sum(1) == 4).all()


@pytest.mark.parametrize("offset,e_local", [(0, 32), (96, 32), (-8, 32), (250, 32), (40, 8)])
def test_local_dispatch_invariants(inputs_mod, offset, e_local):
    cfg, logits, bias = _cfg_routing(inputs_mod, 2)
    r = routing.route(logits.numpy(), bias.to(torch.float32).numpy(), cfg.rsf)
    d = routing.local_dispatch(r["ids"], r["weights"], offset, e_local)
    le = r["ids"] - offset
    local = (le >= 0) & (le < e_local)
    assert d["counts"].sum() == local.sum() == d["offsets"][-1]
    tok = d["route_token"] & 0x7FFFFFFF
    single = d["route_token"] < 0  # bit 31: the token's only local route
    for e in range(e_local):
        rows = tok[d["offsets"][e]:d["offsets"][e + 1]]
        assert (np.diff(rows) > 0).all()  # token order
        assert set(rows.tolist()) == set(np.nonzero((le == e).any(1))[0].tolist())
    for t in range(r["ids"].shape[0]):
        rr = d["token_route"][t]
        n = int(local[t].sum())
        assert (rr[n:] == -1).all() and (rr[:n] >= 0).all() and (np.diff(rr[:n]) > 0).all()
        assert (tok[rr[:n]] == t).all()
        assert (single[rr[:n]] == (n == 1)).all()
