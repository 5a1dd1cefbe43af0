"""GPU parity for the integer/index parts: generator, weight pack, routing and
dispatch -- all bit-exact against the oracle and the golden fixtures."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import pack as opack
from oracle import routing

pytestmark = pytest.mark.gpu


def test_device_generator_matches_host(ops, cuda):
    for seed, stream, n in [(1, 5, 1 << 20), (0x15642001, 7, 3 * 7168 + 5)]:
        t = torch.empty(n, dtype=torch.uint8, device=cuda)
        ops.fill_normal_e4m3_(t, seed, stream)
        assert np.array_equal(t.cpu().numpy(), ops.host_normal_e4m3(n, seed, stream))


# Measured bound on the FP8 MFMA's block-sum error, relative to sum |a*b|
# over the 128 products (the instruction does not round the exact sum to
# fp32; see test_mfma_block_sum_accuracy).  The parity gates use it.
MFMA_REL_BOUND = 2.5e-4


@pytest.mark.parametrize("dist", ["full_range", "normal"])
def test_mfma_block_sum_accuracy(capi, lib, cuda, dist):
    import ctypes

    from oracle.numerics import E4M3_TABLE, e4m3_encode

    n = 4096
    rng = np.random.default_rng(11)
    if dist == "full_range":
        codes = rng.integers(0, 256, size=(2, n, 16, 128), dtype=np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0  # no NaN encodings
    else:
        codes = e4m3_encode(rng.standard_normal((2, n, 16, 128)).astype(np.float32))
    a, b = torch.from_numpy(codes[0]).to(cuda), torch.from_numpy(codes[1]).to(cuda)
    d = torch.empty((n, 16, 16), dtype=torch.float32, device=cuda)
    capi.check(lib.moe_mfma_tiles(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                  ctypes.c_void_p(d.data_ptr()), n, None), "moe_mfma_tiles")
    got = d.cpu().numpy().astype(np.float64)
    A, B = torch.from_numpy(E4M3_TABLE[codes[0]]), torch.from_numpy(E4M3_TABLE[codes[1]])
    exact = torch.bmm(A, B.transpose(1, 2)).numpy()
    mag = torch.bmm(A.abs(), B.abs().transpose(1, 2)).numpy()
    rel = np.abs(got - exact) / np.maximum(mag, 1e-30)
    rn = np.mean(got == exact.astype(np.float32))
    print(f"[mfma] {dist}: worst |err|/sum|ab| = {rel.max():.3e}, equal to RN32(exact): {rn:.4f}", flush=True)
    assert rel.max() <= MFMA_REL_BOUND


def test_mfma_ceiling_probe(capi, lib, cuda):
    """The bench's MFMA-rate probe: finite sums, and per-workgroup counter
    ticks whose ratio is a plausible shader clock."""
    import ctypes

    grid, iters = 16, 64
    out = torch.full((grid * 512,), float("nan"), dtype=torch.float32, device=cuda)
    clocks = torch.zeros(grid * 2, dtype=torch.int64, device=cuda)
    capi.check(lib.moe_mfma_ceiling(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(clocks.data_ptr()), iters,
                                    grid, None), "moe_mfma_ceiling")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    c = clocks.view(grid, 2).cpu()
    assert bool((c > 0).all())
    mhz = 100.0 * c[:, 1].sum().item() / c[:, 0].sum().item()
    print(f"[mfma ceiling probe] mean shader clock {mhz:.0f} MHz", flush=True)
    assert 300.0 < mhz < 4000.0


def test_pack_matches_oracle_permutation(ops, cuda):
    g = torch.Generator(device="cpu").manual_seed(5)
    w13 = torch.randint(0, 256, (2, 4096, 7168), dtype=torch.uint8, generator=g)
    w2 = torch.randint(0, 256, (2, 7168, 2048), dtype=torch.uint8, generator=g)
    p13 = ops.pack_w13(w13.to(cuda))
    p2 = ops.pack_w2(w2.to(cuda))
    assert np.array_equal(p13.cpu().view(torch.uint8).numpy().reshape(-1), opack.pack_w13(w13.numpy()).reshape(-1))
    assert np.array_equal(p2.cpu().view(torch.uint8).numpy().reshape(-1), opack.pack_w2(w2.numpy()).reshape(-1))
    assert torch.equal(ops.unpack_w13(p13).cpu(), w13)
    assert torch.equal(ops.unpack_w2(p2).cpu(), w2)


def test_pack_roundtrip_full_size(ops, inputs_mod, cuda):
    inp = inputs_mod.make_config_inputs(1, device=cuda)
    w13 = inp["gemm1_weights"].view(torch.uint8)
    w2 = inp["gemm2_weights"].view(torch.uint8)
    p13, p2 = ops.pack_w13(inp["gemm1_weights"]), ops.pack_w2(inp["gemm2_weights"])
    assert p13.numel() * 4 == w13.numel() and p2.numel() * 4 == w2.numel()
    assert torch.equal(ops.unpack_w13(p13), w13)
    assert torch.equal(ops.unpack_w2(p2), w2)
    # spot-check the layout formula on the packed bytes
    pb = p13.view(torch.uint8).view(32, 16, 56, 16, 2, 64, 16)
    rng = np.random.default_rng(0)
    for _ in range(64):
        e, nb, kb, t, h, lane, b = (int(rng.integers(0, m)) for m in (32, 16, 56, 16, 2, 64, 16))
        row = (t & 1) * 2048 + nb * 128 + 16 * (t >> 1) + (lane & 15)
        col = kb * 128 + 32 * (lane >> 4) + 16 * h + b
        assert int(pb[e, nb, kb, t, h, lane, b]) == int(w13[e, row, col])


def _gpu_route(ops, logits, bias, rsf, offset, e_local, cuda):
    return ops.route(logits.to(cuda).contiguous(), bias.to(torch.float32).reshape(-1).to(cuda).contiguous(),
                     rsf, offset, e_local)


@pytest.mark.parametrize("idx", [0, 1, 2, 3, 4])
def test_routing_bit_exact(ops, inputs_mod, cuda, idx):
    cfg = inputs_mod.CONFIGS[idx]
    small = inputs_mod.host_tensors(cfg)
    logits, bias = small["routing_logits"], small["routing_bias"]
    print(f"[route] config {idx} T={cfg.T}", flush=True)
    got = _gpu_route(ops, logits, bias, cfg.rsf, cfg.local_expert_offset, 32, cuda)
    ids = got["topk_ids"].cpu().numpy()
    w = got["topk_w"].cpu().numpy()
    fx = np.load(GOLDEN / f"routing_cfg{idx}.npz")
    assert np.array_equal(ids, fx["ids"]), "top-8 sets differ from the reference's routing"
    ref = routing.route(logits.numpy(), bias.to(torch.float32).numpy(), cfg.rsf)
    assert np.array_equal(ids, ref["ids"])
    assert np.array_equal(w.view(np.uint32), ref["weights"].view(np.uint32)), "weights not bit-exact vs oracle"
    d = routing.local_dispatch(ref["ids"], ref["weights"], cfg.local_expert_offset, 32)
    assert np.array_equal(got["counts"].cpu().numpy(), d["counts"])
    assert np.array_equal(got["offsets"].cpu().numpy(), d["offsets"])
    R = int(d["offsets"][-1])
    assert np.array_equal(got["route_token"].cpu().numpy()[:R], d["route_token"])
    assert np.array_equal(got["route_weight"].cpu().numpy()[:R].view(np.uint32), d["route_weight"].view(np.uint32))
    assert np.array_equal(got["token_route"].cpu().numpy(), d["token_route"])


@pytest.mark.parametrize("T,offset,e_local,seed", [(1, 0, 32, 1), (3, 0, 32, 2), (5, -8, 32, 3), (77, 250, 32, 4),
                                                    (130, 40, 8, 5), (2049, 224, 32, 6), (64, 300, 32, 7),
                                                    (3000, 17, 5, 11), (16384, 0, 32, 12),
                                                    (16385, 0, 32, 8), (40000, 96, 32, 9), (70001, 0, 5, 10)])
def test_routing_edge_cases(ops, cuda, T, offset, e_local, seed):
    """Routing and dispatch against the oracle, bit for bit.  Up to T = 16384
    (256 64-token chunks) one launch counts and places, with a grid barrier
    between the two; above that the count, scan and place kernels run."""
    rng = np.random.default_rng(seed)
    logits = torch.from_numpy((rng.standard_normal((T, 256)) * 2).astype(np.float32))
    bias = torch.from_numpy((rng.standard_normal(256) * 0.1).astype(np.float32))
    got = _gpu_route(ops, logits, bias, 1.7, offset, e_local, cuda)
    ref = routing.route(logits.numpy(), bias.numpy(), 1.7)
    assert np.array_equal(got["topk_ids"].cpu().numpy(), ref["ids"])
    assert np.array_equal(got["topk_w"].cpu().numpy().view(np.uint32), ref["weights"].view(np.uint32))
    d = routing.local_dispatch(ref["ids"], ref["weights"], offset, e_local)
    R = int(d["offsets"][-1])
    assert np.array_equal(got["offsets"].cpu().numpy(), d["offsets"])
    assert np.array_equal(got["route_token"].cpu().numpy()[:R], d["route_token"])
    assert np.array_equal(got["token_route"].cpu().numpy(), d["token_route"])


def test_routing_many_ties(ops, cuda):
    """Logits and bias from three and two levels: most biased scores tie,
    inside a lane's four experts, across lanes and across groups, so the
    top-8 cut falls inside runs of equal keys (taken in ascending expert
    order) and the group ranking meets equal scores."""
    rng = np.random.default_rng(77)
    T = 512
    logits = torch.from_numpy(rng.integers(0, 3, size=(T, 256)).astype(np.float32))
    bias = torch.from_numpy((rng.integers(0, 2, size=256) * 0.5).astype(np.float32))
    got = _gpu_route(ops, logits, bias, 2.5, 0, 32, cuda)
    ref = routing.route(logits.numpy(), bias.numpy(), 2.5)
    assert np.array_equal(got["topk_ids"].cpu().numpy(), ref["ids"])
    assert np.array_equal(got["topk_w"].cpu().numpy().view(np.uint32), ref["weights"].view(np.uint32))


def test_routing_exact_ties(ops, cuda):
    logits = torch.zeros((4, 256), dtype=torch.float32)
    logits[1, 100:140] = 1.0  # equal values straddling two groups
    bias = torch.zeros(256)
    got = _gpu_route(ops, logits, bias, 1.0, 0, 32, cuda)
    ref = routing.route(logits.numpy(), bias.numpy(), 1.0)
    assert np.array_equal(got["topk_ids"].cpu().numpy(), ref["ids"])
    assert got["topk_ids"][0].tolist() == list(range(8))
