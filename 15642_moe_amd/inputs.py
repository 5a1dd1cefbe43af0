"""Synthetic inputs for the five benchmark configurations.

Every tensor comes from a counter-based generator (splitmix64 finaliser of
seed, stream and element index), so any slice regenerates bit-identically on
any machine:

* e4m3 tensors (hidden states, W13, W2): Irwin-Hall sum of the four 16-bit
  fields of one hash, times fp32(sqrt(3)/65536) -> ~N(0,1), RNE-encoded.  Made
  on the GPU by ``moe_fill_normal_e4m3`` (or on the CPU by its host twin);
  ``normal_e4m3_numpy`` is the executable specification both are tested
  against.
* fp32 tensors (logits, bias, scales) are small and made on the host with
  exact integer arithmetic and single IEEE operations (numpy float32/float64).

Distributions follow the benchmark definition: logits ~N(0,1) fp32 [T,256];
bias bf16 [256] ~N(0,0.1) (config 4: +3.0 on local experts 0-3, 0 elsewhere);
hidden ~N(0,1) e4m3 with scale ~U(0.01,0.05) [56,T]; W13/W2 ~N(0,1) e4m3 with
scales ~U(0.001,0.01); routed_scaling_factor 2.5.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

from .geometry import E_GLOBAL, E_LOCAL, G1_BLOCKS, H, H_BLOCKS, I_BLOCKS, I_DIM

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15
E4M3_SCALE_BITS = 0x37DDB3D7  # fp32(sqrt(3) / 65536)

# Stream ids, one per tensor.
S_LOGITS, S_BIAS, S_HIDDEN, S_HIDDEN_SCALE, S_W13, S_W13_SCALE, S_W2, S_W2_SCALE = range(1, 9)


@dataclass(frozen=True)
class Config:
    idx: int
    name: str
    T: int
    local_expert_offset: int
    skewed: bool
    seed: int
    rsf: float = 2.5


CONFIGS = {
    0: Config(0, "cpu_plumbing_T16", 16, 0, False, 0x15642000),
    1: Config(1, "decode_T64", 64, 0, False, 0x15642001),
    2: Config(2, "mid_prefill_T1024_off96", 1024, 96, False, 0x15642002),
    3: Config(3, "large_prefill_T8192", 8192, 0, False, 0x15642003),
    4: Config(4, "skewed_T4096", 4096, 0, True, 0x15642004),
}


# --------------------------------------------------------------------------- hashing
def _mix64_int(z: int) -> int:
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> int:
    return _mix64_int((seed * GOLDEN + stream) & M64)


def hash_u64(seed: int, stream: int, n: int, first: int = 0) -> np.ndarray:
    idx = np.arange(first, first + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(stream_key(seed, stream)) + idx * np.uint64(GOLDEN))


# --------------------------------------------------------------------------- encoders
def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> OCP E4M3FN bytes, round-to-nearest-even, overflow/NaN -> 0x7F
    (written from the OCP 8-bit floating point specification)."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    s = ((b >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    a = b & np.uint32(0x7FFFFFFF)
    r = a + np.uint32(0x7FFFF) + ((a >> np.uint32(20)) & np.uint32(1))
    normal = (((r >> np.uint32(23)) - np.uint32(120)) << np.uint32(3)) | ((r >> np.uint32(20)) & np.uint32(7))
    small = np.where(a < np.uint32(0x3C800000), a, np.uint32(0))
    sub = np.rint(small.view(np.float32) * np.float32(512.0)).astype(np.uint32)
    out = np.where(a >= np.uint32(0x3C800000), normal, sub)
    out = np.where(a > np.uint32(0x43E80000), np.uint32(0x7F), out)
    return (out.astype(np.uint8) | s).astype(np.uint8)


def bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


# --------------------------------------------------------------------------- samplers
def normal_e4m3_numpy(seed: int, stream: int, n: int, first: int = 0) -> np.ndarray:
    """Executable specification of the e4m3 ~N(0,1) sequence."""
    h = hash_u64(seed, stream, n, first)
    m = np.uint64(0xFFFF)
    S = (h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m) + (h >> np.uint64(48))
    z = (S.astype(np.int64) - 131070).astype(np.float32) * np.uint32(E4M3_SCALE_BITS).view(np.float32)
    return e4m3_encode(z)


def normal_f32(seed: int, stream: int, n: int) -> np.ndarray:
    """~N(0,1) fp32: Irwin-Hall of four 32-bit uniforms (two hashes per value)."""
    h = hash_u64(seed, stream, 2 * n).reshape(n, 2)
    lo = np.uint64(0xFFFFFFFF)
    S = ((h[:, 0] & lo) + (h[:, 0] >> np.uint64(32)) + (h[:, 1] & lo) + (h[:, 1] >> np.uint64(32))).astype(np.int64)
    z = (S - 2 * 0xFFFFFFFF).astype(np.float64) * float.fromhex("0x1.bb67ae8584caap-32")
    return z.astype(np.float32)


def uniform_f32(seed: int, stream: int, n: int, lo: float, hi: float) -> np.ndarray:
    """U(lo, hi) fp32 = lo + (hi - lo) * u, u = 24 hash bits * 2^-24, fp32 ops."""
    u = (hash_u64(seed, stream, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0**-24)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    return (lo32 + (hi32 - lo32) * u).astype(np.float32)


# --------------------------------------------------------------------------- configs
def host_tensors(cfg: Config) -> dict:
    """The small tensors of a config, as CPU torch tensors."""
    T = cfg.T
    logits = normal_f32(cfg.seed, S_LOGITS, T * E_GLOBAL).reshape(T, E_GLOBAL)
    if cfg.skewed:
        bias32 = np.zeros(E_GLOBAL, dtype=np.float32)
        lo = cfg.local_expert_offset
        bias32[lo:lo + 4] = 3.0
    else:
        bias32 = (normal_f32(cfg.seed, S_BIAS, E_GLOBAL) * np.float32(0.1)).astype(np.float32)
    bias = torch.from_numpy(bf16_rne_bits(bias32).view(np.int16).copy()).view(torch.bfloat16)
    return dict(
        routing_logits=torch.from_numpy(logits),
        routing_bias=bias,
        hidden_states_scale=torch.from_numpy(uniform_f32(cfg.seed, S_HIDDEN_SCALE, H_BLOCKS * T, 0.01, 0.05)
                                             .reshape(H_BLOCKS, T)),
        gemm1_weights_scale=torch.from_numpy(uniform_f32(cfg.seed, S_W13_SCALE, E_LOCAL * G1_BLOCKS * H_BLOCKS,
                                                         0.001, 0.01).reshape(E_LOCAL, G1_BLOCKS, H_BLOCKS)),
        gemm2_weights_scale=torch.from_numpy(uniform_f32(cfg.seed, S_W2_SCALE, E_LOCAL * H_BLOCKS * I_BLOCKS,
                                                         0.001, 0.01).reshape(E_LOCAL, H_BLOCKS, I_BLOCKS)),
    )


def _e4m3_tensor(shape, seed, stream, device) -> torch.Tensor:
    n = int(np.prod(shape))
    if torch.device(device).type == "cuda":
        from . import ops

        t = torch.empty(n, dtype=torch.uint8, device=device)
        ops.fill_normal_e4m3_(t, seed, stream)
    else:
        from . import ops

        t = torch.from_numpy(ops.host_normal_e4m3(n, seed, stream))
    return t.view(torch.float8_e4m3fn).view(shape)


def make_config_inputs(cfg_or_idx, device: str = "cuda") -> dict:
    """All ten north-star inputs of a config, on `device`."""
    cfg = CONFIGS[cfg_or_idx] if isinstance(cfg_or_idx, int) else cfg_or_idx
    small = host_tensors(cfg)
    out = {k: v.to(device) for k, v in small.items()}
    out["hidden_states"] = _e4m3_tensor((cfg.T, H), cfg.seed, S_HIDDEN, device)
    out["gemm1_weights"] = _e4m3_tensor((E_LOCAL, 2 * I_DIM, H), cfg.seed, S_W13, device)
    out["gemm2_weights"] = _e4m3_tensor((E_LOCAL, H, I_DIM), cfg.seed, S_W2, device)
    out["local_expert_offset"] = cfg.local_expert_offset
    out["routed_scaling_factor"] = cfg.rsf
    order = ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale", "gemm1_weights",
             "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale", "local_expert_offset",
             "routed_scaling_factor")
    return {k: out[k] for k in order}


def expert_weights_host(cfg: Config, experts) -> tuple[np.ndarray, np.ndarray]:
    """Host copies of W13/W2 (uint8) for the given local experts only."""
    from . import ops

    per13, per2 = 2 * I_DIM * H, H * I_DIM
    w13 = np.stack([ops.host_normal_e4m3(per13, cfg.seed, S_W13, first_index=e * per13) for e in experts])
    w2 = np.stack([ops.host_normal_e4m3(per2, cfg.seed, S_W2, first_index=e * per2) for e in experts])
    return w13.reshape(len(experts), 2 * I_DIM, H), w2.reshape(len(experts), H, I_DIM)


def sha256(t) -> str:
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu().contiguous().view(torch.uint8).numpy()
    return hashlib.sha256(np.ascontiguousarray(t).tobytes()).hexdigest()
