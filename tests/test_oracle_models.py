"""Pins for the CPU forward models: the real reference's recorded output,
closed forms that fix every scale index and the SwiGLU orientation, and the
expected gap between the fp32 reference and the FP8-requant kernel model."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import moe_cpu
from oracle.numerics import e4m3_encode
from parity import bf16_to_f64, stats


@pytest.fixture(scope="module")
def cfg0_cpu(inputs_mod):
    return inputs_mod.make_config_inputs(0, device="cpu")


def test_reference_model_reproduces_reference_run(cfg0_cpu, inputs_mod):
    """Bit-exact against reference.run's recorded output at config 0."""
    fx = np.load(GOLDEN / "ref_output_cfg0.npz")
    assert str(fx["w13_sha256"]) == inputs_mod.sha256(cfg0_cpu["gemm1_weights"])
    assert str(fx["hidden_sha256"]) == inputs_mod.sha256(cfg0_cpu["hidden_states"])
    out = moe_cpu.forward_reference(cfg0_cpu, routing="torch")
    bits = out.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, fx["out_bits"])


def test_reference_model_with_oracle_routing_close(cfg0_cpu):
    fx = np.load(GOLDEN / "ref_output_cfg0.npz")
    out = moe_cpu.forward_reference(cfg0_cpu, routing="oracle")
    s = stats(out, fx["out_bits"])
    assert s["rel_l2"] < 1e-5  # same sets; weights differ only in summation order


def test_full_dequant_baseline_matches_reference(cfg0_cpu):
    fx = np.load(GOLDEN / "ref_output_cfg0.npz")
    out = moe_cpu.forward_full_dequant(cfg0_cpu)
    assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16), fx["out_bits"])


def test_kernel_model_vs_reference_model(cfg0_cpu):
    km = moe_cpu.kernel_model(cfg0_cpu)
    ref = moe_cpu.forward_reference(cfg0_cpu, ids=km["ids"], weights=km["weights"])
    s = stats(km["out_bits"], ref)
    # FP8 requantisation of the SwiGLU output costs a few percent, never zero
    assert 1e-3 < s["rel_l2"] < 6e-2
    assert np.array_equal(bf16_to_f64(km["out_bits"]) == 0, bf16_to_f64(ref) == 0)


# --------------------------------------------------------------------------- one-hot closed forms
E4M3_ONE, E4M3_TWO = 0x38, 0x40


def _one_hot_problem():
    """Two tokens, one local expert; every nonzero sits in a distinct 128-block
    so a wrong scale index changes the answer."""
    T, H, I = 2, 7168, 2048
    kb = (5, 41)              # hidden K-blocks used by tokens 0 and 1
    col = (kb[0] * 128 + 3, kb[1] * 128 + 77)
    nb, n_local = 9, 21       # I-block and column inside it
    n = nb * 128 + n_local
    ib, h = nb, 30 * 128 + 100  # W2: input column n lies in I-block nb; output row h in H-block 30
    hidden = np.zeros((T, H), np.uint8)
    hidden[0, col[0]] = E4M3_ONE
    hidden[1, col[1]] = E4M3_TWO
    hs = (1.0 + np.arange(56 * T, dtype=np.float32).reshape(56, T) * np.float32(0.25)).astype(np.float32)
    w13 = np.zeros((1, 2 * I, H), np.uint8)
    w13[0, n, col[0]] = E4M3_ONE          # gate row n
    w13[0, I + n, col[0]] = E4M3_TWO      # up row I+n
    w13[0, n, col[1]] = E4M3_TWO
    w13[0, I + n, col[1]] = E4M3_ONE
    s13 = (np.float32(2.0) ** -(np.arange(32 * 56) % 9).astype(np.float32)).reshape(1, 32, 56).astype(np.float32)
    s13 = (s13 * (1 + np.arange(32 * 56).reshape(1, 32, 56) % 5).astype(np.float32)).astype(np.float32)
    w2 = np.zeros((1, H, I), np.uint8)
    w2[0, h, n] = E4M3_ONE
    s2 = (np.float32(0.5) + np.arange(56 * 16, dtype=np.float32).reshape(1, 56, 16) / np.float32(64)).astype(np.float32)
    inputs = {
        "routing_logits": torch.zeros((T, 256)),
        "routing_bias": torch.zeros(256),
        "hidden_states": torch.from_numpy(hidden).view(torch.float8_e4m3fn),
        "hidden_states_scale": torch.from_numpy(hs),
        "gemm1_weights": torch.from_numpy(w13).view(torch.float8_e4m3fn),
        "gemm1_weights_scale": torch.from_numpy(s13),
        "gemm2_weights": torch.from_numpy(w2).view(torch.float8_e4m3fn),
        "gemm2_weights_scale": torch.from_numpy(s2),
        "local_expert_offset": 0,
        "routed_scaling_factor": 1.0,
    }
    ids = np.tile(np.arange(8, dtype=np.int32), (T, 1))
    weights = np.tile(np.array([0.75] + [0.0] * 7, np.float32), (T, 1))
    # closed form in float64: token t uses hidden block kb[t]
    expect = np.zeros((T, H))
    for t, (a, wg, wu) in enumerate([(1.0, 1.0, 2.0), (2.0, 2.0, 1.0)]):
        k = kb[t]
        gate = a * wg * hs[k, t] * s13[0, nb, k]
        up = a * wu * hs[k, t] * s13[0, 16 + nb, k]
        c = gate * up / (1.0 + np.exp(-up))     # silu on the up half (rows I..2I-1)
        expect[t, h] = 0.75 * c * 1.0 * s2[0, h // 128, ib]
    return inputs, ids, weights, expect, h


def test_reference_model_one_hot_closed_form():
    inputs, ids, weights, expect, h = _one_hot_problem()
    out = bf16_to_f64(moe_cpu.forward_reference(inputs, ids=ids, weights=weights))
    np.testing.assert_allclose(out[:, h], expect[:, h], rtol=2 ** -8)
    assert np.count_nonzero(out) == 2


def test_kernel_model_one_hot_closed_form():
    inputs, ids, weights, expect, h = _one_hot_problem()
    km = moe_cpu.kernel_model(inputs, ids=ids, weights=weights, keep_intermediates=True)
    out = bf16_to_f64(km["out_bits"])
    np.testing.assert_allclose(out[:, h], expect[:, h], rtol=2 ** -8)
    assert np.count_nonzero(out) == 2
    ex = km["experts"][0]
    # a lone nonzero in its 128-block quantises to +-448 exactly
    assert np.count_nonzero(ex["Cq"]) == 2
    assert set(np.unique(ex["Cq"][ex["Cq"] != 0]).tolist()) <= {0x7E, 0xFE}
    assert np.all(ex["Cs"][:, [b for b in range(16) if b != 9]] == np.float32(1e-8))


def test_one_hot_detects_swapped_gate_up():
    """Planted mistake on the CPU: SwiGLU on the gate half changes the answer."""
    inputs, ids, weights, expect, h = _one_hot_problem()
    hs, s13 = inputs["hidden_states_scale"].numpy(), inputs["gemm1_weights_scale"].numpy()
    k = 5
    gate = hs[k, 0] * s13[0, 9, k]
    up = 2.0 * hs[k, 0] * s13[0, 25, k]
    wrong = up * gate / (1.0 + np.exp(-gate))
    right = gate * up / (1.0 + np.exp(-up))
    assert abs(wrong - right) > 1e-3 * abs(right)
    assert abs(expect[0, h] / (0.75 * inputs["gemm2_weights_scale"].numpy()[0, 30, 9]) - right) < 1e-6 * abs(right)


def test_c_requant_scale_formula():
    rng = np.random.default_rng(0)
    a = e4m3_encode(rng.standard_normal((3, 7168)).astype(np.float32))
    w = e4m3_encode(rng.standard_normal((4096, 7168)).astype(np.float32))
    cq, cs, c = moe_cpu.stage1_model(a, np.full((3, 56), 0.02, np.float32), w, np.full((32, 56), 0.004, np.float32))
    amax = np.abs(c.reshape(3, 16, 128)).max(2)
    np.testing.assert_array_equal(cs, np.maximum((amax / np.float32(448)).astype(np.float32), np.float32(1e-8)))
    deq = (moe_cpu.E4M3_TABLE[cq].reshape(3, 16, 128) * cs[:, :, None]).reshape(3, 2048)
    assert np.all(np.abs(deq - c) <= np.abs(c) * 2 ** -4 + np.repeat(cs, 128, 1) * 2 ** -9)
