"""moe_forward_noalloc under HIP graph capture (helpers; the tests are in
test_zz_no_alloc.py).  A forward captured into a torch.cuda.CUDAGraph must
replay to exactly moe_forward's output after the graph's input tensors are
overwritten with new activations and routing logits; eager work (a fill of
the output, the reference forward) runs between the replays.  Run as a
script, one case in this process: python graph_noalloc.py T warm(0|1)."""

from __future__ import annotations

import ctypes
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from conftest import pkg  # noqa: E402

E_LOCAL = 32


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32).contiguous()


def run_graph_case(T: int, warm: bool, rounds: int = 3, seed: int = 900) -> None:
    """Capture moe_forward_noalloc at T tokens (after one eager call when
    `warm`, else as the process's first forward call: the first call on the
    device looks up the library's scratch array, and every forward kernel is
    launched for the first time inside the capture), then replay `rounds`
    times over new inputs, each against the eager moe_forward, bit for bit."""
    layer, ops, capi = pkg("moe_layer"), pkg("ops"), pkg("capi")
    lib = capi.load()
    dev = torch.device("cuda:0")
    base = layer.build_moe_inputs(T=T, device="cuda", seed=seed)
    p13, p2 = ops.pack_w13(base["gemm1_weights"]), ops.pack_w2(base["gemm2_weights"])
    rsf, offset = float(base["routed_scaling_factor"]), int(base["local_expert_offset"])
    # the tensors the captured forward reads (rewritten in place before each replay)
    hidden = base["hidden_states"].clone()
    hscale = _f32(base["hidden_states_scale"]).clone()
    logits = _f32(base["routing_logits"]).clone()
    s13, s2 = _f32(base["gemm1_weights_scale"]), _f32(base["gemm2_weights_scale"])
    bias = _f32(base["routing_bias"]).reshape(-1).clone()
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    ptrs = [ctypes.c_void_p(t.data_ptr()) for t in (hidden, hscale, p13, s13, p2, s2, logits, bias)]

    def forward(stream: torch.cuda.Stream) -> None:
        rc = lib.moe_forward_noalloc(*ptrs, rsf, offset, T, E_LOCAL, ctypes.c_void_p(out.data_ptr()),
                                     ctypes.c_void_p(stream.cuda_stream))
        capi.check(rc, "moe_forward_noalloc")

    if warm:
        forward(torch.cuda.current_stream(dev))
        torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()

    gen = torch.Generator(device="cuda")
    for r in range(rounds):
        gen.manual_seed(seed + 1 + r)
        hidden.copy_((torch.rand(T, 7168, generator=gen, device=dev) * 2 - 1).to(torch.float8_e4m3fn))
        hscale.copy_(torch.rand(56, T, generator=gen, device=dev) * 0.1 + 0.01)
        logits.copy_(torch.randn(T, 256, generator=gen, device=dev))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = ops.moe_forward(hidden, hscale, p13, s13, p2, s2, logits, bias, rsf, offset)
        torch.cuda.synchronize()
        print(f"[graph] T={T} warm={warm} replay {r}", flush=True)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {r} differs from moe_forward"
        assert float(out.float().abs().sum()) > 0
    del graph


if __name__ == "__main__":
    run_graph_case(int(sys.argv[1]), bool(int(sys.argv[2])))
    print("[graph] ok", flush=True)
