"""Comparison helpers shared by the parity tests (no tests here)."""

from __future__ import annotations

import numpy as np
import torch


def bf16_to_f64(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu()
        if x.dtype == torch.bfloat16:
            x = x.view(torch.int16).numpy().view(np.uint16)
        else:
            return x.to(torch.float64).numpy()
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return (x.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)
    return x.astype(np.float64)


def stats(got, ref) -> dict:
    g, r = bf16_to_f64(got), bf16_to_f64(ref)
    d = np.abs(g - r)
    norm = np.linalg.norm(r)
    return {
        "rel_l2": float(np.linalg.norm(g - r) / norm) if norm > 0 else float(np.linalg.norm(g)),
        "max_abs": float(d.max()) if d.size else 0.0,
        "ref_absmax": float(np.abs(r).max()) if r.size else 0.0,
        "bitwise_equal_frac": float(np.mean(g == r)) if g.size else 1.0,
    }


def reference_tolerance_bad(got, ref, atol: float = 1e-2, rtol: float = 2e-2) -> int:
    """Elements failing the reference test's gate |d| <= atol + rtol*|ref|
    (tests/test_moe.py:21-40)."""
    g, r = bf16_to_f64(got), bf16_to_f64(ref)
    return int(np.count_nonzero(np.abs(g - r) > atol + rtol * np.abs(r)))


def scaled_bad(got, ref, rel_rms: float, rtol: float) -> int:
    """Scale-aware elementwise gate |d| <= rel_rms*rms(ref) + rtol*|ref|; the
    fixed 1e-2 atol of the reference test is vacuous when outputs are ~1e-5."""
    g, r = bf16_to_f64(got), bf16_to_f64(ref)
    rms = np.sqrt(np.mean(r * r)) if r.size else 0.0
    return int(np.count_nonzero(np.abs(g - r) > rel_rms * rms + rtol * np.abs(r)))


def report(tag: str, s: dict) -> None:
    print(f"[parity] {tag}: " + " ".join(f"{k}={v:.3e}" if isinstance(v, float) else f"{k}={v}" for k, v in s.items()),
          flush=True)
