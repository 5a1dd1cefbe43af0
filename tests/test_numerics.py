"""Oracle codecs against torch's CPU casts (exhaustive where feasible) and the
shared sigmoid evaluation against the float64 closed form."""

from __future__ import annotations

import numpy as np
import torch

from oracle import numerics


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encode_matches_torch_over_fp32_range():
    # every 61st fp32 bit pattern with |x| in [0, 464], both signs (~2x19M values)
    lo, hi = 0x00000000, 0x43E80000
    for start in range(lo, hi + 1, 1 << 27):
        bits = np.arange(start, min(start + (1 << 27), hi + 1), 61, dtype=np.uint32)
        x = bits.view(np.float32)
        for v in (x, -x):
            assert np.array_equal(numerics.e4m3_encode(v), _torch_e4m3(v)), hex(start)


def test_e4m3_encode_rounding_boundaries():
    # all midpoints between adjacent finite codes (ties to even) and neighbours
    vals = np.sort(np.unique(numerics.E4M3_TABLE[np.isfinite(numerics.E4M3_TABLE)]))
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)
    probes = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    assert np.array_equal(numerics.e4m3_encode(probes), _torch_e4m3(probes))


def test_e4m3_saturation():
    x = np.array([448.0, 463.9, 464.0, 464.1, 1e9, np.inf, -500.0], dtype=np.float32)
    assert numerics.e4m3_encode(x, saturate=True).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE]
    assert numerics.e4m3_encode(x).tolist()[:4] == [0x7E, 0x7E, 0x7E, 0x7F]


def test_e4m3_decode_table_matches_torch():
    t = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    ours = numerics.E4M3_TABLE
    nan = np.isnan(t)
    assert np.array_equal(nan, np.isnan(ours))
    assert np.array_equal(t[~nan], ours[~nan])
    assert nan.sum() == 2  # 0x7F, 0xFF


def test_package_encoder_is_the_oracle_encoder(inputs_mod):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1 << 20) * rng.choice([1e-3, 1.0, 100.0], 1 << 20)).astype(np.float32)
    assert np.array_equal(inputs_mod.e4m3_encode(x), numerics.e4m3_encode(x))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(1 << 20) * 10.0 ** rng.integers(-30, 30, 1 << 20)).astype(np.float32)
    bits = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32)
    y = bits.view(np.float32)
    y = y[np.isfinite(y)]
    for v in (x, y):
        want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(numerics.bf16_bits(v), want)


def test_sigmoid_within_two_ulp_of_exact():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1 << 20) * 3).astype(np.float32)
    ours = numerics.sigmoid(x)
    exact = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    ulps = np.abs(ours.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 2  # three fp32 roundings: exp, 1 + e, 1 / d
    assert np.mean(ulps == 0) > 0.5
    # the formula is the one torch evaluates, up to its exp: most values agree
    agree = np.mean(ours == torch.sigmoid(torch.from_numpy(x)).numpy())
    assert agree > 0.9


def test_sigmoid_known_values():
    x = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 100.0, -100.0], dtype=np.float32)
    s = numerics.sigmoid(x)
    assert s[0] == np.float32(0.5)
    assert s[3] == np.float32(1.0 / (1.0 + np.float32(np.exp(-20.0))))
    assert s[5] == np.float32(1.0) and s[6] == np.float32(0.0)  # 1 / (1 + inf)
    assert abs(float(s[1]) - 1 / (1 + np.exp(-1.0))) < 1e-7
