"""The producer in front of the path: router GEMM + dynamic FP8 activation
quantisation (moe_router_quant), against oracle/upstream.py.

CPU: the oracle's known answers, its agreement with torch's own
float8_e4m3fn cast, the dequantisation round trip, one-hot router rows, and
the packed router layout.  GPU: codes and scales bit-exact, logits within the
fp32 accumulation bound of the exact sums, deterministic, and the produced
inputs drive moe_forward to the same bits as the oracle's.
"""

from __future__ import annotations

import math
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import upstream as up
from oracle.numerics import bf16_bits, bf16_value, e4m3_decode, e4m3_encode

H, E, NB = 7168, 256, 56
LOGIT_REL = 2e-5  # |gpu - exact| / sum|x*w|: 224 fp32 accumulations of 32-term MFMA sums


def _hidden_bits(T: int, seed: int) -> np.ndarray:
    """bf16 activations with a spread of block magnitudes, a zero block, a
    one-hot block and values that land on e4m3 subnormals."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, NB, 128)).astype(np.float32)
    x *= np.exp2(rng.integers(-20, 8, size=(T, NB, 1))).astype(np.float32)
    if T > 0:
        x[0, 3] = 0.0
        x[0, 4] = 0.0
        x[0, 4, 17] = -5.5
        x[-1, 7, :64] *= np.float32(2.0**-12)
    return bf16_bits(x.reshape(T, H))


def _router_bits(seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return bf16_bits((rng.standard_normal((E, H)) * 0.02).astype(np.float32))


# --------------------------------------------------------------------------- CPU: oracle
def test_act_quant_known_answers():
    x = np.zeros((2, H), dtype=np.float32)
    x[0, :128] = np.linspace(-3.0, 1.5, 128, dtype=np.float32)   # block max |x| = 3 at column 0
    x[0, 128:256] = 0.75                                            # constant block
    x[1, 300] = 2.0**-30                                            # a lone tiny value
    codes, scale = up.act_quant(bf16_bits(x))
    assert scale.shape == (NB, 2)
    assert scale[0, 0] == np.float32(3.0) / np.float32(448.0)
    assert codes[0, 0] == 0xFE                                      # -448
    assert (codes[0, 128:256] == 0x7E).all() and scale[1, 0] == np.float32(0.75) / np.float32(448.0)
    assert scale[5, 0] == np.float32(1e-8) and (codes[0, 640:768] == 0).all()   # zero block
    assert scale[2, 1] == np.float32(1e-8)                          # 2^-30 / 448 < 1e-8: floor
    q = np.float32(2.0**-30) / np.float32(1e-8)                     # ~0.107, a normal e4m3 value
    assert codes[1, 300] == e4m3_encode(np.array([q], np.float32))[0] and 0 < codes[1, 300] < 0x7E


def test_act_quant_matches_torch_cast():
    """The oracle equals torch's own e4m3 cast of the clamped quotient."""
    bits = _hidden_bits(9, 1)
    codes, scale = up.act_quant(bits)
    x = torch.from_numpy(bf16_value(bits)).reshape(9, NB, 128)
    s = torch.from_numpy(scale.T.copy())[:, :, None]
    q = (x / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).reshape(9, H).numpy()
    assert np.array_equal(codes, q)


def test_act_quant_round_trip():
    bits = _hidden_bits(17, 2)
    codes, scale = up.act_quant(bits)
    x = bf16_value(bits).astype(np.float64).reshape(17, NB, 128)
    back = e4m3_decode(codes).reshape(17, NB, 128) * scale.T[:, :, None].astype(np.float64)
    s = scale.T[:, :, None].astype(np.float64)
    # half an e4m3 step: 2^-4 relative in the normal range, 2^-10 * scale below it
    tol = np.maximum(np.abs(x) * 2.0**-4, s * 2.0**-10) * (1 + 1e-6)
    assert (np.abs(back - x) <= tol).all()
    # a block's maximum maps to +-448 unless the 1e-8 scale floor applies
    amax = np.abs(x).max(axis=2)
    hit = (amax > 0) & (s[:, :, 0] > np.float32(1e-8))
    assert hit.sum() > 100
    assert np.array_equal(np.abs(back).max(axis=2)[hit], 448.0 * s[:, :, 0][hit])


def test_router_logits_one_hot_rows():
    w = _router_bits(3)
    x = np.zeros((4, H), dtype=np.float32)
    cols = [0, 127, 4096, 7167]
    for t, c in enumerate(cols):
        x[t, c] = 1.0
    got = up.router_logits(bf16_bits(x), w)
    assert np.array_equal(got, bf16_value(w)[:, cols].T.astype(np.float64))


def test_pack_router_layout():
    w = _router_bits(4)
    p = up.pack_router(w)
    assert p.shape == (56, 4, 16, 64, 8)
    for kb, ks, t, lane in [(0, 0, 0, 0), (7, 1, 3, 18), (55, 3, 15, 63)]:
        k = kb * 128 + ks * 32 + 8 * (lane // 16)
        assert np.array_equal(p[kb, ks, t, lane], w[16 * t + lane % 16, k:k + 8])
    assert np.array_equal(up.unpack_router(p), w)


def _quotient_checker(tmp_path) -> Path:
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    exe = tmp_path / "quotient_exhaustive"
    src = Path(__file__).with_name("quotient_exhaustive.c")
    subprocess.run([gcc, "-O2", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"], check=True)
    return exe


def test_quantiser_quotient_exhaustive(tmp_path):
    """The quantiser's block scale RN(amax/448) comes from a reciprocal
    product plus one FMA correction, and it divides by the scale as
    reciprocal times x plus one correction, with the reciprocal from
    v_rcp_f32 (documented as accurate to 1 ulp) (upstream.hip quant_scale,
    quot).  tests/quotient_exhaustive.c checks the scale bit for bit for
    every finite bf16 amax.  It checks the codes for every bf16 element each
    amax bounds (1.07e9 pairs, all of the kernel's input domain) with each
    reciprocal within 1 ulp of 1/s, and every bf16 x (infinities and NaNs
    included) in a block whose amax is +inf.  Every code must equal that of
    the IEEE quotient x / s.  The amax range is split over 8 processes of
    about equal work."""
    exe = _quotient_checker(tmp_path)
    top = 0x7F80
    edges = [round(top * math.sqrt(i / 8)) for i in range(9)]
    procs = [subprocess.Popen([str(exe), str(lo), str(hi)], stdout=subprocess.PIPE, text=True)
             for lo, hi in zip(edges[:-1], edges[1:])]
    cases = 0
    for p in procs:
        out, _ = p.communicate(timeout=900)
        assert p.returncode == 0, out
        assert out.strip().endswith(" 0 code differences") and "scale: 0 differences" in out, out
        cases += int(out.split("):")[1].split()[0])
    # every (amax, |x| <= amax, sign) pair with three reciprocals each, and
    # every bf16 x in a block whose amax is +inf
    assert cases == 3 * sum(2 * ab + 2 for ab in range(top)) + 65536


def test_quantiser_quotient_checker_rejects_plain_reciprocal(tmp_path):
    """Planted mistake: the quotient without its correction step, RN(x * RN(1/s)),
    gives other codes (first found at amax 1.5234375, bf16 0x3FC3)."""
    exe = _quotient_checker(tmp_path)
    bad = subprocess.run([str(exe), "16323", "16324", "plain"], capture_output=True, text=True)
    assert bad.returncode == 1 and "code differs" in bad.stdout
    good = subprocess.run([str(exe), "16323", "16324"], capture_output=True, text=True)
    assert good.returncode == 0, good.stdout


# --------------------------------------------------------------------------- GPU
def _to_dev(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).to(dev).view(torch.bfloat16)


@pytest.fixture(scope="module")
def router(ops, cuda):
    w = _router_bits(11)
    packed = ops.pack_router(_to_dev(w, cuda))
    return w, packed


@pytest.mark.gpu
def test_pack_router_matches_oracle(ops, cuda, router):
    w, packed = router
    got = packed.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, up.pack_router(w))
    assert np.array_equal(ops.unpack_router(packed).view(torch.int16).cpu().numpy().view(np.uint16), w)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 7, 64, 100, 1000, 4096, 4097, 6000])
def test_router_quant_parity(ops, cuda, router, T):
    w, packed = router
    bits = _hidden_bits(T, 100 + T)
    logits, hq, hs = ops.router_quant(_to_dev(bits, cuda), packed)
    torch.cuda.synchronize()
    codes, scale = up.act_quant(bits)
    print(f"router_quant T={T}", flush=True)
    assert np.array_equal(hq.view(torch.uint8).cpu().numpy(), codes)
    assert np.array_equal(hs.cpu().numpy(), scale)
    exact = up.router_logits(bits, w)
    bound = up.logits_bound(bits, w)
    err = np.abs(logits.cpu().numpy().astype(np.float64) - exact)
    assert (err <= LOGIT_REL * bound + 1e-30).all(), float((err / np.maximum(bound, 1e-300)).max())
    again = ops.router_quant(_to_dev(bits, cuda), packed)[0]
    assert torch.equal(again, logits)  # K parts are added in a fixed order


@pytest.mark.gpu
def test_router_quant_full_size_sampled(ops, cuda, router):
    w, packed = router
    T = 8192
    bits = _hidden_bits(T, 5)
    logits, hq, hs = ops.router_quant(_to_dev(bits, cuda), packed)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 63, 64, 4095, 8190, 8191])
    codes, scale = up.act_quant(bits[rows])
    assert np.array_equal(hq.view(torch.uint8)[rows].cpu().numpy(), codes)
    assert np.array_equal(hs[:, rows].cpu().numpy(), scale)
    exact = up.router_logits(bits[rows], w)
    err = np.abs(logits[rows].cpu().numpy().astype(np.float64) - exact)
    assert (err <= LOGIT_REL * up.logits_bound(bits[rows], w) + 1e-30).all()


@pytest.mark.gpu
def test_router_quant_feeds_forward(ops, inputs_mod, cuda, router):
    """The produced tensors are moe_forward inputs: the forward over them
    equals, bit for bit, the forward over the oracle's codes and scales with
    the same logits."""
    w, packed = router
    inp = inputs_mod.make_config_inputs(1, device=cuda)
    T = 64
    bits = _hidden_bits(T, 21)
    logits, hq, hs = ops.router_quant(_to_dev(bits, cuda), packed)
    codes, scale = up.act_quant(bits)
    p13, p2 = ops.pack_w13(inp["gemm1_weights"]), ops.pack_w2(inp["gemm2_weights"])
    f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
    args = (p13, f32(inp["gemm1_weights_scale"]), p2, f32(inp["gemm2_weights_scale"]))
    bias = f32(inp["routing_bias"]).reshape(-1)
    out = ops.moe_forward(hq, hs, *args, logits, bias, 2.5, 0)
    ref = ops.moe_forward(torch.from_numpy(codes).to(cuda).view(torch.float8_e4m3fn),
                          torch.from_numpy(scale).to(cuda), *args, logits, bias, 2.5, 0)
    assert torch.equal(out, ref)
    assert out.abs().sum() > 0
