"""Write the golden fixtures under tests/golden/ (run in the build container,
which has /root/reference; the fixtures then travel with the repo).

  routing_cfg{0..4}.npz   top-8 sets and weights from the reference's routing
                          op sequence (reference/moe_ref.py:81-107, evaluated
                          by oracle.moe_cpu.route_torch on the CPU), plus
                          SHA-256 of the logits/bias they came from, and the
                          decision margins of the numpy oracle.
  ref_output_cfg0.npz     bf16 output of the real reference.run
                          (reference/moe_ref.py) at config 0 (T=16), and
  ref_output_builder_T8.npz  at the reference builder's own distributions
                          (moe_layer.build_moe_inputs, T=8, seed=8, CPU).
                          Only these need the reference import: nothing else
                          fixes its exact output bits.

    python tests/golden/make_golden.py [--skip-reference]
"""

from __future__ import annotations

import argparse
import importlib
import json
import sys
import time
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

pkg = importlib.import_module("15642_moe_amd")
inputs_mod = importlib.import_module("15642_moe_amd.inputs")
moe_layer = importlib.import_module("15642_moe_amd.moe_layer")
from oracle import moe_cpu, routing  # noqa: E402

REFERENCE_DIR = Path("/root/reference")


def routing_fixtures() -> dict:
    summary = {}
    for idx, cfg in inputs_mod.CONFIGS.items():
        small = inputs_mod.host_tensors(cfg)
        logits, bias = small["routing_logits"], small["routing_bias"]
        topk_idx, dense = moe_cpu.route_torch(logits, bias, cfg.rsf)
        ids_t = torch.sort(topk_idx, dim=1).values.numpy().astype(np.int32)
        w_t = torch.gather(dense, 1, torch.sort(topk_idx, dim=1).values).numpy().astype(np.float32)
        r = routing.route(logits.numpy(), bias.to(torch.float32).numpy(), cfg.rsf)
        mism = np.nonzero((r["ids"] != ids_t).any(axis=1))[0]
        np.savez_compressed(
            HERE / f"routing_cfg{idx}.npz",
            ids=ids_t,
            weights=w_t,
            expert_margin=r["expert_margin"].astype(np.float32),
            group_margin=r["group_margin"].astype(np.float32),
            logits_sha256=np.array(inputs_mod.sha256(logits)),
            bias_sha256=np.array(inputs_mod.sha256(bias)),
            T=np.int32(cfg.T),
            offset=np.int32(cfg.local_expert_offset),
        )
        local = ((ids_t >= cfg.local_expert_offset) & (ids_t < cfg.local_expert_offset + 32))
        summary[cfg.name] = dict(
            T=cfg.T,
            oracle_vs_torch_mismatched_tokens=[int(t) for t in mism],
            local_routes=int(local.sum()),
            hit_experts=int(len(np.unique(ids_t[local]))),
            max_weight_rel_diff=float(np.max(np.abs(r["weights"] - w_t) / np.abs(w_t))),
            min_expert_margin=float(r["expert_margin"].min()),
            min_group_margin=float(r["group_margin"].min()),
        )
        print(cfg.name, summary[cfg.name], flush=True)
    return summary


def _reference_run():
    # The reference tree is read-only: importing it must not leave
    # __pycache__ bytecode behind in it.
    sys.dont_write_bytecode = True
    sys.path.insert(0, str(REFERENCE_DIR))
    ref = importlib.import_module("reference")
    return ref.run


def _config_inputs_cpu(idx: int) -> dict:
    return inputs_mod.make_config_inputs(idx, device="cpu")


def reference_outputs() -> dict:
    run = _reference_run()
    out = {}
    t0 = time.time()
    inp = _config_inputs_cpu(0)
    y = run(**inp)
    np.savez_compressed(HERE / "ref_output_cfg0.npz", out_bits=y.view(torch.int16).numpy().view(np.uint16),
                        hidden_sha256=np.array(inputs_mod.sha256(inp["hidden_states"])),
                        w13_sha256=np.array(inputs_mod.sha256(inp["gemm1_weights"])),
                        w2_sha256=np.array(inputs_mod.sha256(inp["gemm2_weights"])))
    out["cfg0"] = dict(seconds=time.time() - t0, absmax=float(y.float().abs().max()),
                       nonzero_rows=int((y.float().abs().sum(1) > 0).sum()))
    print("cfg0 reference output", out["cfg0"], flush=True)
    del inp, y
    t0 = time.time()
    inp = moe_layer.build_moe_inputs(T=8, device="cpu", seed=8)
    y = run(**inp)
    np.savez_compressed(HERE / "ref_output_builder_T8.npz", out_bits=y.view(torch.int16).numpy().view(np.uint16),
                        w13_sha256=np.array(inputs_mod.sha256(inp["gemm1_weights"])))
    out["builder_T8"] = dict(seconds=time.time() - t0, absmax=float(y.float().abs().max()))
    print("builder T8 reference output", out["builder_T8"], flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-reference", action="store_true")
    args = ap.parse_args()
    torch.set_num_threads(max(1, torch.get_num_threads()))
    summary = {"routing": routing_fixtures()}
    if not args.skip_reference:
        summary["reference"] = reference_outputs()
    (HERE / "golden_summary.json").write_text(json.dumps(summary, indent=1) + "\n")


if __name__ == "__main__":
    main()
