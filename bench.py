#!/usr/bin/env python3
"""moe_forward benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,3,4] [--no-cpu-baseline]
                    [--no-headline] [--no-upstream] [--no-sweep] [--sweep-steps S]

A step is one moe_forward (route, dispatch, GEMM1+SwiGLU+FP8 requant,
GEMM2, combine) over one batch with pre-packed weights already resident in
HBM; the one-time pack is timed separately.  The headline line is the decode
configuration (T=64); the other configurations are timed
too and reported under "configs".  Per-kernel durations come from HIP events
recorded on the launch stream between the kernels (moe_forward_timed), and
give the roofline figure of the dominant kernel.  Each configuration is also
timed through moe_layer.run_custom, the drop-in path the reference's own
benchmark times (pack-cache lookups, fp32 casts, then ops.moe_forward).  The
CPU baseline times the oracle's restatement of reference/moe_ref.py (full
fp32 dequant, per-expert fp32 GEMMs) on the host, on whole forwards of each
configuration's batch (a bounded number per configuration).  Under
"upstream", the producer of the forward's inputs (moe_router_quant: router
GEMM + dynamic FP8 activation quantisation from bf16 hidden states) is timed
at each configuration's T.  Under "reference_sweep" (and as latency-only
"reference_T<T>" entries under "configs"), run_custom is timed at the
reference benchmark's own T points with its builder's inputs
(bench/bench_moe.py:18-20,101-118).

Prints one JSON line on stdout; progress goes to stderr.  --no-headline
times only the listed configurations (for per-configuration kernel traces)
and prints a line with their records only.
"""

from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense FP8 MFMA, TFLOP/s
METRIC = "moe_forward latency (µs) at T=64/1024/8192; FP8 MFMA util % and HBM GB/s"
STAGES = ("route", "dispatch", "gemm1_swiglu_quant", "gemm2", "combine")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _traffic_from_profiles(config_name: str) -> dict:
    """HBM bytes per launch of the dominant kernel, the kernel and the commit
    it was measured at, from the committed rocprofv3 PMC summary
    (profiles/traffic_<workload>.txt: 'traffic_bytes_per_launch: N',
    'dominant_kernel: ...', 'commit: ...'); values None when absent."""
    rec = {"traffic": None, "traffic_kernel": None, "traffic_commit": None}
    p = REPO / "profiles" / f"traffic_{config_name}.txt"
    if not p.exists():
        return rec
    for line in p.read_text().splitlines():
        key, _, val = line.partition(":")
        if key == "traffic_bytes_per_launch":
            rec["traffic"] = float(val)
        elif key == "dominant_kernel":
            rec["traffic_kernel"] = val.strip()
        elif key == "commit":
            rec["traffic_commit"] = val.strip()
    return rec


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="1,2,3,4", help="benchmark configs to time (headline: 1)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=12.0, help="CPU-baseline wall time per configuration")
    ap.add_argument("--no-headline", action="store_true",
                    help="time only the listed configs (no headline config 1, no summary line)")
    ap.add_argument("--no-upstream", action="store_true", help="skip the moe_router_quant timing")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the reference benchmark's own T sweep (run_custom at its builder's inputs)")
    ap.add_argument("--sweep-steps", type=int, default=20, help="timed run_custom calls per T of the sweep")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run one plain 512 MiB device copy (the known-size reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE into bytes) and exit")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} requested). "
              "Expert-parallel sharding is a design note only; run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    if args.calibrate_copy:
        return _calibrate_copy(torch)
    inputs_mod = importlib.import_module("15642_moe_amd.inputs")
    ops = importlib.import_module("15642_moe_amd.ops")
    capi = importlib.import_module("15642_moe_amd.capi")
    geo = importlib.import_module("15642_moe_amd.geometry")
    lib = capi.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    cfg_ids = [int(c) for c in args.configs.split(",") if c.strip()]
    if 1 not in cfg_ids and not args.no_headline:
        cfg_ids = [1] + cfg_ids
    moe_layer = importlib.import_module("15642_moe_amd.moe_layer")
    results = {}
    cpu_runs = {}

    for idx in cfg_ids:
        cfg = inputs_mod.CONFIGS[idx]
        log(f"config {idx} {cfg.name}: generating inputs")
        inp = inputs_mod.make_config_inputs(idx, device=dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        p13 = ops.pack_w13(inp["gemm1_weights"])
        p2 = ops.pack_w2(inp["gemm2_weights"])
        torch.cuda.synchronize()
        pack_us = (time.perf_counter() - t0) * 1e6

        f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
        args_fwd = (inp["hidden_states"], f32(inp["hidden_states_scale"]), p13, f32(inp["gemm1_weights_scale"]), p2,
                    f32(inp["gemm2_weights_scale"]), f32(inp["routing_logits"]), f32(inp["routing_bias"]).reshape(-1))
        T, E = cfg.T, 32
        rsf, off = float(cfg.rsf), int(cfg.local_expert_offset)

        # routing statistics -> algorithmic work (exact counts at this seed)
        r = ops.route(args_fwd[6], args_fwd[7], rsf, off, E)
        counts = r["counts"].cpu()
        routes = int(counts.sum())
        hit = int((counts > 0).sum())
        alg_bytes = hit * geo.BYTES_PER_EXPERT + T * geo.BYTES_PER_TOKEN + geo.BYTES_FIXED
        alg_flops = routes * geo.FLOPS_PER_ROUTE
        w13_bytes = 2 * geo.I_DIM * geo.H + geo.G1_BLOCKS * geo.H_BLOCKS * 4
        w2_bytes = geo.H * geo.I_DIM + geo.H_BLOCKS * geo.I_BLOCKS * 4
        stage_bytes = {
            "gemm1_swiglu_quant": hit * w13_bytes + T * (geo.H + geo.H_BLOCKS * 4) + routes * (geo.I_DIM + 64),
            "gemm2": hit * w2_bytes + routes * (geo.I_DIM + 64 + geo.H * 4),
        }
        stage_flops = {"gemm1_swiglu_quant": routes * 2 * geo.H * 2 * geo.I_DIM, "gemm2": routes * 2 * geo.I_DIM * geo.H}

        out = torch.empty((T, geo.H), dtype=torch.bfloat16, device=dev)
        ws_bytes = int(lib.moe_workspace_bytes(T, E))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        stream = torch.cuda.current_stream(dev)
        ptrs = [ctypes.c_void_p(t.data_ptr()) for t in args_fwd]
        sptr = ctypes.c_void_p(stream.cuda_stream)

        def fwd():
            rc = lib.moe_forward(*ptrs, rsf, off, T, E, ctypes.c_void_p(ws.data_ptr()), ws_bytes,
                                 ctypes.c_void_p(out.data_ptr()), sptr)
            if rc:
                capi.check(rc, "moe_forward")

        for _ in range(args.warmup):
            fwd()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.steps):
            fwd()
        end.record(stream)
        torch.cuda.synchronize()
        total_ms = start.elapsed_time(end)
        lat_us = total_ms * 1e3 / args.steps

        # per-kernel durations: events between the launches, on the launch stream
        n_ev = capi.FORWARD_EVENTS
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(n_ev)] for _ in range(args.steps)]
        for row in evs:
            for e in row:
                e.record(stream)  # creates the underlying HIP event
        torch.cuda.synchronize()
        for row in evs:
            handles = (ctypes.c_void_p * n_ev)(*[ctypes.c_void_p(e.cuda_event) for e in row])
            rc = lib.moe_forward_timed(*ptrs, rsf, off, T, E, ctypes.c_void_p(ws.data_ptr()), ws_bytes,
                                       ctypes.c_void_p(out.data_ptr()), sptr, handles, n_ev)
            capi.check(rc, "moe_forward_timed")
        torch.cuda.synchronize()
        stage_us = {}
        for i, name in enumerate(STAGES):
            stage_us[name] = sum(row[i].elapsed_time(row[i + 1]) for row in evs) * 1e3 / args.steps
        if T <= geo.DECODE_MAX_T:
            # the decode path runs its dispatch inside GEMM1: the event pair
            # around the dispatch stage brackets no kernel (only event cost)
            stage_us["dispatch"] = None

        # the drop-in path the reference benchmark times: moe_layer.run_custom
        # (its pack cache is filled by the warm-up calls)
        kw = {k: inp[k] for k in ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
                                  "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale")}
        kw.update(local_expert_offset=off, routed_scaling_factor=rsf)
        for _ in range(max(args.warmup, 1)):
            moe_layer.run_custom(ops, **kw)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            moe_layer.run_custom(ops, **kw)
        end.record(stream)
        torch.cuda.synchronize()
        run_custom_us = start.elapsed_time(end) * 1e3 / args.steps
        moe_layer._packed_weight_cache.clear()

        rec = {
            "T": T,
            "local_expert_offset": off,
            "latency_us": round(lat_us, 2),
            "run_custom_us": round(run_custom_us, 2),
            "local_routes": routes,
            "hit_experts": hit,
            "alg_bytes": alg_bytes,
            "alg_flops": alg_flops,
            "hbm_gbs": round(alg_bytes / (lat_us * 1e-6) / 1e9, 1),
            "hbm_frac": round(alg_bytes / (lat_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "mfma_util": round(alg_flops / (lat_us * 1e-6) / 1e12 / FP8_PEAK_TFLOPS, 4),
            "stage_us": {k: (None if v is None else round(v, 2)) for k, v in stage_us.items()},
            "stage_gbs": {k: round(stage_bytes[k] / (stage_us[k] * 1e-6) / 1e9, 1) for k in stage_bytes},
            "stage_tflops": {k: round(stage_flops[k] / (stage_us[k] * 1e-6) / 1e12, 2) for k in stage_flops},
            "stage_alg_bytes": stage_bytes,
            "pack_us_one_time": round(pack_us, 1),
        }
        results[cfg.name] = rec
        log(f"config {idx}: {json.dumps(rec)}")
        if not args.no_cpu_baseline:
            cpu_runs[cfg.name] = _cpu_baseline(
                {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}, cfg, lat_us,
                args.cpu_budget_s)
        del inp, p13, p2, args_fwd, out, ws, evs, kw
        torch.cuda.empty_cache()

    sweep = [] if args.no_sweep or args.no_headline else _reference_sweep(torch, moe_layer, args.sweep_steps)
    upstream = [] if args.no_upstream or args.no_headline else [
        _time_upstream(torch, lib, dev, inputs_mod.CONFIGS[i].T, args.steps) for i in cfg_ids]
    # last: its full-power MFMA launches leave the GPU hot for what follows
    ceiling = _mfma_ceiling(torch, lib, dev, capi)
    for rec in results.values():
        rec["stage_frac_of_mfma_ceiling"] = {k: round(v / ceiling["tflops"], 4) for k, v in rec["stage_tflops"].items()}
    # the reference benchmark's own T points, latency only, beside the configs
    for rec in sweep:
        results[f"reference_T{rec['T']}"] = {
            **rec, "latency_us": rec["run_custom_us"],
            "workload": "reference builder inputs (moe_layer.build_moe_inputs), timed through moe_layer.run_custom"}
    if args.no_headline:
        print(json.dumps({"metric": METRIC, "configs": results, "mfma_ceiling": ceiling,
                          "cpu_baseline_per_config": cpu_runs or None}), flush=True)
        return 0

    head = results[inputs_mod.CONFIGS[1].name]
    dom = max(("gemm1_swiglu_quant", "gemm2"), key=lambda k: head["stage_us"][k])
    achieved = head["stage_alg_bytes"][dom] / (head["stage_us"][dom] * 1e-6) / 1e9
    roofline = {
        "kernel": dom,
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        **_traffic_from_profiles(inputs_mod.CONFIGS[1].name),
        "launch_us": head["stage_us"][dom],
        "alg_bytes_per_launch": head["stage_alg_bytes"][dom],
    }

    cpu_baseline = None
    hname = inputs_mod.CONFIGS[1].name
    if hname in cpu_runs:
        c = cpu_runs[hname]
        cpu_baseline = {
            "value": c["us"],
            "unit": "us per moe_forward (T=64)",
            "cores": c["cores"],
            "kind": "port",
            "sample": c["sample"],
            "cpu": _cpu_model(),
            "gpu_speedup": c["gpu_speedup"],
            "per_config": cpu_runs,
        }

    line = {
        "metric": METRIC,
        "value": head["latency_us"],
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["latency_us"] / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic: counter-based generator, BASELINE distributions (N(0,1) e4m3 weights/activations)",
        "config": {
            "workload": "decode_T64 (BASELINE configs[1]): DeepSeek-V3 MoE layer, T=64, H=7168, I=2048, "
                        "256 experts / 32 local (offset 0), top-8 of 8 groups (top-4 groups), rsf 2.5",
            "T": 64,
            "local_routes": head["local_routes"],
            "hit_experts": head["hit_experts"],
            "parallelism": "single GPU, 32 local experts",
        },
        "hbm_gbs": head["hbm_gbs"],
        "mfma_util": head["mfma_util"],
        "roofline": roofline,
        "cpu_baseline": cpu_baseline,
        "configs": results,
        "reference_sweep": sweep,
        "mfma_ceiling": ceiling,
        "upstream": upstream,
    }
    print(json.dumps(line), flush=True)
    return 0


# The reference benchmark's T points and its timing loop (bench/bench_moe.py:18-20,35-46,101-118): at
# each T, the reference builder's inputs (seed 0: U(-1,1) e4m3 activations and weights, scales
# U(0.01, 0.11), zero bias, rsf 1.0) timed through the drop-in run_custom, 10 warm-up calls first.
REFERENCE_T_VALUES = (1, 4, 32, 64, 256, 2048, 4096, 8192, 16384)


def _reference_sweep(torch, moe_layer, steps: int) -> list:
    """Latency of moe_layer.run_custom at each of the reference benchmark's T
    values with its own builder's inputs; FLOPs counted as the reference does
    (local routes x FLOPS_PER_ROUTE, bench/bench_moe.py:29-32,103-104)."""
    geo = importlib.import_module("15642_moe_amd.geometry")
    ops = moe_layer._load_custom_ops()
    stream = torch.cuda.current_stream()
    out = []
    for T in REFERENCE_T_VALUES:
        inp = moe_layer.build_moe_inputs(T=T, device="cuda")
        routes = int(ops.route(inp["routing_logits"].to(torch.float32).contiguous(),
                               inp["routing_bias"].to(torch.float32).contiguous(),
                               float(inp["routed_scaling_factor"]), int(inp["local_expert_offset"]))["counts"].sum())
        for _ in range(10):
            moe_layer.run_custom(ops, **inp)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            moe_layer.run_custom(ops, **inp)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / steps
        rec = {"T": T, "local_routes": routes, "run_custom_us": round(us, 2),
               "tflops": round(routes * geo.FLOPS_PER_ROUTE / (us * 1e-6) / 1e12, 1), "steps": steps}
        log(f"reference sweep: {json.dumps(rec)}")
        out.append(rec)
        moe_layer._packed_weight_cache.clear()
        del inp
        torch.cuda.empty_cache()
    return out


def _mfma_ceiling(torch, lib, dev, capi) -> dict:
    """The FP8 MFMA rate this GPU sustains with nothing but MFMAs in flight
    (moe_mfma_ceiling: one 512-thread workgroup per CU, 4 independent
    32x32x64 MFMA chains per wave, ~2 ms per launch), and the mean shader
    clock it ran at.  Dense FP8 work on every CU draws enough power that the
    clock drops well below its maximum, so this, not the published peak, is
    the rate a compute-bound kernel can approach; the prefill GEMMs'
    stage_frac_of_mfma_ceiling compares them with it.  Median of 5 timed
    launches after one warm-up launch."""
    grid = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 4000
    flops = grid * 8 * iters * 4 * 2 * 32 * 32 * 64
    out = torch.empty(grid * 512, dtype=torch.float32, device=dev)
    clocks = torch.zeros(grid * 2, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    rates, mhz = [], []
    for rep in range(6):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        capi.check(lib.moe_mfma_ceiling(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(clocks.data_ptr()), iters,
                                        grid, ctypes.c_void_p(stream.cuda_stream)), "moe_mfma_ceiling")
        end.record(stream)
        torch.cuda.synchronize()
        if rep == 0:
            continue
        c = clocks.view(grid, 2).cpu().double()
        rates.append(flops / (start.elapsed_time(end) * 1e-3) / 1e12)
        mhz.append(100.0 * c[:, 1].sum().item() / c[:, 0].sum().item())
    if not bool(torch.isfinite(out).all()):
        raise RuntimeError("moe_mfma_ceiling produced non-finite sums")
    rates.sort()
    mhz.sort()
    rec = {"kernel": "mfma_ceiling_kernel (fp8 32x32x64, register operands, no memory traffic)",
           "tflops": round(rates[len(rates) // 2], 1), "clock_mhz": round(mhz[len(mhz) // 2]),
           "frac_of_peak": round(rates[len(rates) // 2] / FP8_PEAK_TFLOPS, 4), "workgroups": grid, "iters": iters}
    log(f"mfma ceiling: {json.dumps(rec)}")
    return rec


def _cpu_baseline(inputs_cpu: dict, cfg, gpu_us: float, budget_s: float) -> dict:
    """The oracle's restatement of reference/moe_ref.run (full fp32 dequant,
    per-expert fp32 GEMMs) on whole forwards of one configuration's batch, on
    the host's cores: one warm-up forward, then up to three timed ones
    (fewer only when the next would run past budget_s)."""
    import torch

    from oracle import moe_cpu  # CPU-baseline leg only

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    log(f"cpu baseline: oracle restatement of moe_ref.run, {cfg.name} (T={cfg.T}), {cores} threads")
    times = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        moe_cpu.forward_full_dequant(inputs_cpu)
        times.append(time.perf_counter() - t0)
        log(f"cpu baseline {cfg.name} forward {len(times)}: {times[-1]:.2f} s")
        if len(times) >= 4 or time.perf_counter() + times[-1] > t_end:
            break
    steady = times[1:] if len(times) > 1 else times
    us = sum(steady) / len(steady) * 1e6
    return {
        "us": round(us, 1),
        "T": cfg.T,
        "cores": torch.get_num_threads(),
        "timed_forwards": len(steady),
        "sample": (f"1 warm-up + {len(steady)} timed full forwards of config {cfg.name}" if len(times) > 1
                   else f"1 full forward of config {cfg.name}"),
        "gpu_speedup": round(us / gpu_us, 1),
    }


def _time_upstream(torch, lib, dev, T: int, steps: int) -> dict:
    """moe_router_quant (router GEMM + FP8 activation quant, the producer of
    the forward's inputs) at T tokens: synthetic bf16 hidden states and router
    weight, outputs and workspace allocated once, HIP events around `steps`
    launches on the current stream."""
    ops = importlib.import_module("15642_moe_amd.ops")
    g = torch.Generator(device=dev).manual_seed(0x15642 + T)
    hidden = torch.randn((T, 7168), generator=g, device=dev).to(torch.bfloat16)
    router = (torch.randn((256, 7168), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    packed = ops.pack_router(router)
    logits = torch.empty((T, 256), dtype=torch.float32, device=dev)
    hq = torch.empty((T, 7168), dtype=torch.uint8, device=dev)
    hs = torch.empty((56, T), dtype=torch.float32, device=dev)
    ws_bytes = int(lib.moe_router_workspace_bytes(T))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    vp = ctypes.c_void_p
    argv = (vp(hidden.data_ptr()), vp(packed.data_ptr()), T, vp(ws.data_ptr()), ws_bytes, vp(logits.data_ptr()),
            vp(hq.data_ptr()), vp(hs.data_ptr()), vp(stream.cuda_stream))
    for _ in range(3):
        lib.moe_router_quant(*argv)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        rc = lib.moe_router_quant(*argv)
        if rc:
            importlib.import_module("15642_moe_amd.capi").check(rc, "moe_router_quant")
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / steps
    alg_bytes = T * (7168 * 2 + 7168 + 56 * 4 + 256 * 4) + 256 * 7168 * 2
    rec = {"kernel": "router_quant_kernel", "T": T, "us": round(us, 2), "alg_bytes": alg_bytes,
           "hbm_gbs": round(alg_bytes / (us * 1e-6) / 1e9, 1),
           "tflops": round(2.0 * T * 7168 * 256 / (us * 1e-6) / 1e12, 2)}
    log(f"upstream T={T}: {json.dumps(rec)}")
    del hidden, router, packed, logits, hq, hs, ws
    return rec


def _calibrate_copy(torch) -> int:
    """One device-to-device copy of exactly 512 MiB (read 512 MiB, write
    512 MiB): profiled with --pmc FETCH_SIZE / WRITE_SIZE it gives the factor
    from counter kilobytes to bytes moved."""
    n = 512 << 20
    src = torch.full((n,), 1, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {n} bytes")
    return 0


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor()


if __name__ == "__main__":
    sys.exit(main())
