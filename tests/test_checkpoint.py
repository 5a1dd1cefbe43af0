"""DeepSeek-V3 checkpoint loader (15642_moe_amd/checkpoint.py).

CPU: the tensor-name mapping and the GEMM1 row orientation (up_proj in rows
[0, 2048), gate_proj in rows [2048, 4096)) pinned against DeepSeek's MLP
formula down(silu(gate x) * up x) and the reference's SwiGLU
(reference/moe_ref.py:129-130); single-file, sharded-with-index and
directory-scan checkpoints; shape, dtype, name and range errors.  GPU: the
packed-at-load buffers equal ops.pack_w13 / pack_w2 of the unpacked tensors
bit for bit, and the forward over them equals the forward over the
reference layout.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import pkg

ck = pkg("checkpoint")
I, H = 2048, 7168


def _expert(seed: int):
    """Random e4m3 bytes (no NaN codes) and positive block scales, in the forward's layout."""
    rng = np.random.default_rng(seed)
    def f8(shape):
        b = rng.integers(0, 256, size=shape, dtype=np.uint8)
        b[(b & 0x7F) == 0x7F] = 0x38  # replace NaN codes with 1.0
        return torch.from_numpy(b).view(torch.float8_e4m3fn)
    w13, w2 = f8((2 * I, H)), f8((H, I))
    s13 = torch.from_numpy(rng.uniform(1e-3, 1e-2, size=(32, 56)).astype(np.float32))
    s2 = torch.from_numpy(rng.uniform(1e-3, 1e-2, size=(56, 16)).astype(np.float32))
    return w13, s13, w2, s2


@pytest.fixture(scope="module")
def experts():
    return {5: _expert(1), 6: _expert(2)}


@pytest.fixture(scope="module")
def layer_tensors(experts):
    bias = torch.linspace(-1, 1, 256, dtype=torch.float32)
    router = (torch.arange(256 * H, dtype=torch.float32).reshape(256, H) % 7 - 3).to(torch.bfloat16)
    return bias, router


def _bytes(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def test_orientation_matches_deepseek_mlp(tmp_path):
    """Written by hand in DeepSeek's naming: after loading, the reference's
    SwiGLU over GEMM1 rows equals down(silu(gate x) * up x)."""
    from safetensors.torch import save_file

    rng = np.random.default_rng(3)
    gate = torch.from_numpy(rng.standard_normal((I, H)).astype(np.float32) * 0.05).to(torch.float8_e4m3fn)
    up = torch.from_numpy(rng.standard_normal((I, H)).astype(np.float32) * 0.05).to(torch.float8_e4m3fn)
    down = torch.from_numpy(rng.standard_normal((H, I)).astype(np.float32) * 0.05).to(torch.float8_e4m3fn)
    one = lambda shape: torch.ones(shape, dtype=torch.float32)  # noqa: E731
    L, e = 9, 0
    save_file({
        ck.expert_key(L, e, "gate_proj"): gate, ck.expert_key(L, e, "up_proj"): up, ck.expert_key(L, e, "down_proj"): down,
        ck.expert_key(L, e, "gate_proj", "weight_scale_inv"): one((16, 56)) * 2,
        ck.expert_key(L, e, "up_proj", "weight_scale_inv"): one((16, 56)) * 3,
        ck.expert_key(L, e, "down_proj", "weight_scale_inv"): one((56, 16)) * 5,
        ck.bias_key(L): torch.zeros(256),
    }, str(tmp_path / "model.safetensors"))
    w = ck.load_moe_layer(tmp_path, L, 0, 1, pack=False)
    assert w.router_weight is None and not w.packed
    assert (w.w13_scale[0, :16] == 3).all() and (w.w13_scale[0, 16:] == 2).all() and (w.w2_scale[0] == 5).all()

    x = rng.standard_normal(H)
    f64 = lambda t: t.to(torch.float32).numpy().astype(np.float64)  # noqa: E731
    # DeepSeek-V3 MLP on the dequantised checkpoint weights
    g, u = f64(gate) * 2 @ x, f64(up) * 3 @ x
    want = (f64(down) * 5) @ (g / (1 + np.exp(-g)) * u)
    # the reference's SwiGLU over the loaded GEMM1 rows (moe_ref.py:128-131)
    W13 = f64(w.w13[0]) * np.repeat(w.w13_scale[0].numpy().astype(np.float64), 128, axis=0)[:, :1]
    G1 = W13 @ x
    X1, X2 = G1[:I], G1[I:]
    got = (f64(w.w2[0]) * 5) @ ((X2 / (1.0 + np.exp(-X2))) * X1)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shards", [1, 3])
def test_round_trip_unpacked(tmp_path, experts, layer_tensors, shards):
    bias, router = layer_tensors
    ck.save_moe_layer(tmp_path, 4, experts, bias, router, shards=shards)
    if shards > 1:
        index = json.loads((tmp_path / ck.INDEX_FILE).read_text())
        assert len(set(index["weight_map"].values())) == shards
    w = ck.load_moe_layer(tmp_path, 4, local_expert_offset=5, n_local=2, pack=False)
    for le, e in enumerate((5, 6)):
        w13, s13, w2, s2 = experts[e]
        assert np.array_equal(_bytes(w.w13[le]), _bytes(w13))
        assert np.array_equal(_bytes(w.w2[le]), _bytes(w2))
        assert torch.equal(w.w13_scale[le], s13) and torch.equal(w.w2_scale[le], s2)
    assert torch.equal(w.routing_bias, bias) and torch.equal(w.router_weight, router)


def test_directory_scan_without_index(tmp_path, experts, layer_tensors):
    bias, _ = layer_tensors
    ck.save_moe_layer(tmp_path, 4, experts, bias, None, shards=2)
    (tmp_path / ck.INDEX_FILE).unlink()
    w = ck.load_moe_layer(tmp_path, 4, local_expert_offset=6, n_local=1, pack=False)
    assert np.array_equal(_bytes(w.w13[0]), _bytes(experts[6][0]))


def test_errors(tmp_path, experts, layer_tensors):
    bias, _ = layer_tensors
    ck.save_moe_layer(tmp_path, 4, experts, bias)
    with pytest.raises(KeyError, match="experts.7.up_proj"):
        ck.load_moe_layer(tmp_path, 4, local_expert_offset=6, n_local=2, pack=False)
    with pytest.raises(KeyError, match="layers.3"):
        ck.load_moe_layer(tmp_path, 3, local_expert_offset=5, n_local=1, pack=False)
    with pytest.raises(ValueError):
        ck.load_moe_layer(tmp_path, 4, local_expert_offset=250, n_local=8, pack=False)
    with pytest.raises(ValueError):
        ck.load_moe_layer(tmp_path, 4, local_expert_offset=0, n_local=33, pack=False)
    with pytest.raises(RuntimeError, match="HIP device"):
        ck.load_moe_layer(tmp_path, 4, local_expert_offset=5, n_local=1, device="cpu", pack=True)
    bad = tmp_path / "bad"
    w13, s13, w2, s2 = experts[5]
    ck.save_moe_layer(bad, 4, {5: (w13, s13, w2[:, :1024], s2)}, bias)
    with pytest.raises(ValueError, match="down_proj.weight: expected"):
        ck.load_moe_layer(bad, 4, local_expert_offset=5, n_local=1, pack=False)


@pytest.mark.gpu
def test_packed_load_matches_pack_and_forward(tmp_path, ops, inputs_mod, cuda, experts, layer_tensors):
    bias, router = layer_tensors
    ck.save_moe_layer(tmp_path, 4, experts, bias, router, shards=2)
    w = ck.load_moe_layer(tmp_path, 4, local_expert_offset=5, n_local=2, device=cuda)
    print("checkpoint packed load", flush=True)
    W13 = torch.stack([experts[e][0] for e in (5, 6)]).to(cuda)
    W2 = torch.stack([experts[e][2] for e in (5, 6)]).to(cuda)
    assert torch.equal(w.w13, ops.pack_w13(W13)) and torch.equal(w.w2, ops.pack_w2(W2))
    assert torch.equal(w.w13_scale.cpu(), torch.stack([experts[e][1] for e in (5, 6)]))
    assert torch.equal(w.router_weight.cpu(), router) and w.routing_bias.is_cuda

    inp = inputs_mod.make_config_inputs(1, device=cuda)
    f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
    act = (inp["hidden_states"], f32(inp["hidden_states_scale"]))
    logits = f32(inp["routing_logits"])
    logits[:, 5:7] += 4.0  # make the two loaded experts hit
    s13, s2 = w.w13_scale.contiguous(), w.w2_scale.contiguous()
    rb = f32(inp["routing_bias"]).reshape(-1)  # the loaded linspace bias would steer picks away from experts 5, 6
    out = ops.moe_forward(*act, w.w13, s13, w.w2, s2, logits, rb, 2.5, 5)
    ref = ops.moe_forward(*act, ops.pack_w13(W13), s13, ops.pack_w2(W2), s2, logits, rb, 2.5, 5)
    assert torch.equal(out, ref) and out.abs().sum() > 0


def _normal_expert(seed: int):
    """One expert with the benchmark's distributions (N(0,1) e4m3 weights,
    block scales ~U(1e-3, 1e-2)), in the forward's layout."""
    g = torch.Generator().manual_seed(seed)
    f8 = lambda shape: torch.randn(shape, generator=g).clamp(-448, 448).to(torch.float8_e4m3fn)  # noqa: E731
    u = lambda shape: (torch.rand(shape, generator=g) * 9e-3 + 1e-3).to(torch.float32)  # noqa: E731
    return f8((2 * I, H)), u((32, 56)), f8((H, I)), u((56, 16))


@pytest.mark.gpu
@pytest.mark.parametrize("T", [64, 300])
def test_checkpoint_forward_matches_oracle(tmp_path, inputs_mod, cuda, T):
    """A checkpoint in DeepSeek naming (gate_proj / up_proj / down_proj with
    their weight_scale_inv, gate.e_score_correction_bias) loaded straight into
    the packed layout, run through moe_forward with the loaded routing bias:
    the output matches the CPU oracle on the unpacked load (kernel-semantics
    model and the reference semantics, reference/moe_ref.py:5-136), and for
    sampled tokens the float64 DeepSeek MLP sum_e w_e * down_e(silu(gate_e x) *
    up_e x) evaluated on the checkpoint tensors themselves.  T=64 runs the
    decode kernels, T=300 the prefill tiles."""
    from oracle import moe_cpu
    from parity import bf16_to_f64, reference_tolerance_bad, report, stats

    ops = pkg("ops")
    L, offset, n_local = 7, 64, 3
    experts = {offset + i: _normal_expert(100 + i) for i in range(n_local)}
    bias = torch.from_numpy((np.random.default_rng(5).standard_normal(256) * 0.1).astype(np.float32))
    bias[offset:offset + n_local] += 0.4  # the loaded experts are picked often, not by every token
    ck.save_moe_layer(tmp_path, L, experts, bias, shards=2)
    print(f"[checkpoint] T={T}: loading packed", flush=True)
    w = ck.load_moe_layer(tmp_path, L, local_expert_offset=offset, n_local=n_local, device=cuda)
    wc = ck.load_moe_layer(tmp_path, L, local_expert_offset=offset, n_local=n_local, pack=False)
    assert torch.equal(w.routing_bias.cpu(), bias)

    cfg = inputs_mod.Config(200 + T, f"checkpoint_T{T}", T, offset, False, 0x15642200 + T)
    inp = inputs_mod.make_config_inputs(cfg, device=cuda)
    f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
    out = ops.moe_forward(inp["hidden_states"], f32(inp["hidden_states_scale"]), w.w13, w.w13_scale.contiguous(),
                          w.w2, w.w2_scale.contiguous(), f32(inp["routing_logits"]), w.routing_bias, 2.5, offset)
    torch.cuda.synchronize()

    cpu = {
        "routing_logits": inp["routing_logits"].cpu(), "routing_bias": bias,
        "hidden_states": inp["hidden_states"].cpu(), "hidden_states_scale": inp["hidden_states_scale"].cpu(),
        "gemm1_weights": wc.w13, "gemm1_weights_scale": wc.w13_scale,
        "gemm2_weights": wc.w2, "gemm2_weights_scale": wc.w2_scale,
        "local_expert_offset": offset, "routed_scaling_factor": 2.5,
    }
    km = moe_cpu.kernel_model(cpu)
    ids = km["ids"]
    nloc = ((ids >= offset) & (ids < offset + n_local)).sum(1)
    assert nloc.sum() >= T // 2 and (nloc >= 2).any(), "the loaded experts must receive routes"
    ref = moe_cpu.forward_reference(cpu, ids=ids, weights=km["weights"])
    got = bf16_to_f64(out)
    s_km, s_ref = stats(got, bf16_to_f64(km["out_bits"])), stats(got, bf16_to_f64(ref))
    report(f"checkpoint T={T} vs kernel-model", s_km)
    report(f"checkpoint T={T} vs reference", s_ref)
    assert s_km["rel_l2"] <= 5e-3
    assert reference_tolerance_bad(got, bf16_to_f64(ref)) == 0 and s_ref["rel_l2"] <= 6e-2
    assert np.array_equal(got[nloc == 0], np.zeros_like(got[nloc == 0]))

    # float64 DeepSeek MLP on the checkpoint's own tensors, for a few tokens
    from safetensors import safe_open

    def tensor(name):
        for f in tmp_path.glob("*.safetensors"):
            with safe_open(str(f), framework="pt") as h:
                if name in h.keys():
                    return h.get_tensor(name)
        raise KeyError(name)

    def deq(proj, e):
        wt = tensor(ck.expert_key(L, e, proj)).to(torch.float64)
        s = tensor(ck.expert_key(L, e, proj, "weight_scale_inv")).to(torch.float64)
        return wt * s.repeat_interleave(128, 0).repeat_interleave(128, 1)

    mats = {e: (deq("gate_proj", e), deq("up_proj", e), deq("down_proj", e)) for e in experts}
    a = inp["hidden_states"].cpu().to(torch.float64) * \
        inp["hidden_states_scale"].cpu().to(torch.float64).t().repeat_interleave(128, 1)
    toks = [int(t) for t in np.nonzero(nloc)[0][:: max(1, int(np.count_nonzero(nloc)) // 6)]]
    for t in toks:
        want = torch.zeros(H, dtype=torch.float64)
        for k, e in enumerate(ids[t]):
            if e in mats:
                gate, up, down = mats[int(e)]
                g_, u_ = gate @ a[t], up @ a[t]
                want += float(km["weights"][t, k]) * (down @ (g_ / (1 + torch.exp(-g_)) * u_))
        d = got[t] - want.numpy()
        rel = float(np.linalg.norm(d) / np.linalg.norm(want.numpy()))
        print(f"[checkpoint] T={T} token {t} ({int(nloc[t])} loaded experts): rel-L2 vs float64 DeepSeek MLP {rel:.3e}",
              flush=True)
        assert rel <= 6e-2  # FP8 requant of the SwiGLU output costs a few percent
