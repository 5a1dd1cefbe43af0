"""moe_forward_noalloc: the forward over the library's own per-GPU scratch
array, for callers that cannot allocate.  Its output must equal
moe_forward's (same kernels, a caller workspace) bit for bit, on calls in a
row whose second input is smaller than the first (the scratch keeps the
previous call's contents), on both the decode and the prefill kernels; and
captured into a HIP graph (torch.cuda.CUDAGraph), with and without an eager
call first, every replay over new inputs must equal moe_forward bit for
bit."""

from __future__ import annotations

import ctypes
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from conftest import pkg

pytestmark = pytest.mark.gpu


def _noalloc(lib, inp, p13, p2, T, E):
    f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
    keep = [inp["hidden_states"], f32(inp["hidden_states_scale"]), p13, f32(inp["gemm1_weights_scale"]), p2,
            f32(inp["gemm2_weights_scale"]), f32(inp["routing_logits"]), f32(inp["routing_bias"]).reshape(-1)]
    out = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=p13.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(p13.device).cuda_stream)
    rc = lib.moe_forward_noalloc(*[ctypes.c_void_p(t.data_ptr()) for t in keep],
                                 float(inp["routed_scaling_factor"]), int(inp["local_expert_offset"]), T, E,
                                 ctypes.c_void_p(out.data_ptr()), stream)
    pkg("capi").check(rc, "moe_forward_noalloc")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("sizes", [(128, 33), (130, 129)])
def test_noalloc_forward_equals_workspace_forward(cuda, sizes):
    """(128, 33): decode kernels; (130, 129): prefill kernels (dispatch, work
    queues, tile GEMMs), the second call smaller than the first."""
    layer, ops, capi = pkg("moe_layer"), pkg("ops"), pkg("capi")
    lib = capi.load()
    E = 32
    for k, T in enumerate(sizes):
        assert lib.moe_workspace_bytes(T, E) <= lib.moe_noalloc_scratch_bytes()
        inp = layer.build_moe_inputs(T=T, device="cuda", seed=700 + 10 * k + T)
        p13, p2 = ops.pack_w13(inp["gemm1_weights"]), ops.pack_w2(inp["gemm2_weights"])
        print(f"[noalloc] call {k}: T={T}", flush=True)
        got = _noalloc(lib, inp, p13, p2, T, E)
        f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
        want = ops.moe_forward(inp["hidden_states"], f32(inp["hidden_states_scale"]), p13,
                               f32(inp["gemm1_weights_scale"]), p2, f32(inp["gemm2_weights_scale"]),
                               f32(inp["routing_logits"]), f32(inp["routing_bias"]).reshape(-1),
                               float(inp["routed_scaling_factor"]), int(inp["local_expert_offset"]))
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {k} (T={T}) differs"
        assert float(got.float().abs().sum()) > 0
        # the same call again over the scratch the first one left behind
        again = _noalloc(lib, inp, p13, p2, T, E)
        assert torch.equal(again.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_sizes_beyond_its_scratch(cuda):
    capi = pkg("capi")
    lib = capi.load()
    T = 4096
    assert lib.moe_workspace_bytes(T, 32) > lib.moe_noalloc_scratch_bytes()
    null = ctypes.c_void_p(0)
    rc = lib.moe_forward_noalloc(*([null] * 8), 1.0, 0, T, 32, null, null)
    assert rc == capi.MOE_ERR_WORKSPACE
    assert b"moe_forward_noalloc" in lib.moe_last_error()


@pytest.mark.parametrize("T", [64, 130])
def test_noalloc_graph_capture_after_a_call(cuda, T):
    """T=64: decode kernels; T=130: prefill kernels.  One eager call, then
    capture, then replays over new inputs (graph_noalloc.run_graph_case)."""
    from graph_noalloc import run_graph_case

    print(f"[graph] in-process T={T}", flush=True)
    run_graph_case(T, warm=True)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("T", [64, 130])
def test_noalloc_graph_capture_as_first_call(cuda, T):
    """The capture is the process's first forward call (the scratch address
    lookup and every forward kernel's first launch happen inside it): a
    fresh child process runs graph_noalloc.py for this T."""
    script = Path(__file__).resolve().with_name("graph_noalloc.py")
    print(f"[graph] child process T={T}", flush=True)
    res = subprocess.run([sys.executable, str(script), str(T), "0"], capture_output=True, text=True, timeout=540)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0, f"child exited {res.returncode}"
    assert "[graph] ok" in res.stdout
