"""DeepSeek-V3/R1 checkpoint loader for one MoE layer's routed experts.

The reference has no loader: its inputs come from a random builder
(moe_layer.py:45-75), and `run_custom` packs whole `[E, 4096, 7168]` /
`[E, 7168, 2048]` weight tensors on every new tensor (moe_layer.py:77-95),
so a real model would hold each layer's weights twice.  This module reads the
published checkpoint layout (Hugging Face safetensors shards with a
`model.safetensors.index.json` weight map) and writes each local expert
straight into its slot of the packed gfx950 operand buffers, one expert at a
time: device memory peaks at the packed weights plus one expert's staging
copy.

Checkpoint tensors of layer L, expert e (block-scaled FP8, 128x128 blocks,
`weight_scale_inv` being the dequantisation multiplier despite its name):

    model.layers.L.mlp.experts.e.gate_proj.weight            e4m3 [2048, 7168]
    model.layers.L.mlp.experts.e.gate_proj.weight_scale_inv  f32  [16, 56]
    model.layers.L.mlp.experts.e.up_proj.weight              e4m3 [2048, 7168]
    model.layers.L.mlp.experts.e.up_proj.weight_scale_inv    f32  [16, 56]
    model.layers.L.mlp.experts.e.down_proj.weight            e4m3 [7168, 2048]
    model.layers.L.mlp.experts.e.down_proj.weight_scale_inv  f32  [56, 16]
    model.layers.L.mlp.gate.weight                           bf16 [256, 7168]
    model.layers.L.mlp.gate.e_score_correction_bias          f32  [256]

Mapping onto the forward's operands: the reference applies SiLU to GEMM1
rows [I, 2I) and multiplies by rows [0, I) (reference/moe_ref.py:129-130),
and DeepSeek's MLP is down(silu(gate(x)) * up(x)), so

    gemm1_weights[le]       = cat(up_proj.weight, gate_proj.weight)      [4096, 7168]
    gemm1_weights_scale[le] = cat(up_proj.scale,  gate_proj.scale)       [32, 56]
    gemm2_weights[le]       = down_proj.weight                           [7168, 2048]
    gemm2_weights_scale[le] = down_proj.scale                            [56, 16]
    routing_bias            = e_score_correction_bias                    [256]

for le = e - local_expert_offset.  The router weight feeds the input
producer (ops.pack_router / ops.router_quant).  Naming caution: the
reference kernel calls GEMM1 rows [0, I) "gate" and rows [I, 2I) "up"
(kernels/moe.cu:483-487, the scale blocks nb and nb+16), the opposite of
the checkpoint's names for the same rows; the kernels here follow the
reference's naming.

Files are opened with safetensors' own reader (no pickle); nothing in a
checkpoint is executed.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path

import torch

from .geometry import E_GLOBAL, G1_BLOCKS, H, H_BLOCKS, I_BLOCKS, I_DIM, MAX_E_LOCAL, W13_PACKED_SHAPE, W2_PACKED_SHAPE

INDEX_FILE = "model.safetensors.index.json"


def expert_key(layer: int, expert: int, proj: str, what: str = "weight") -> str:
    return f"model.layers.{layer}.mlp.experts.{expert}.{proj}.{what}"


def router_key(layer: int) -> str:
    return f"model.layers.{layer}.mlp.gate.weight"


def bias_key(layer: int) -> str:
    return f"model.layers.{layer}.mlp.gate.e_score_correction_bias"


class Checkpoint:
    """Tensor name -> shard file of a safetensors checkpoint: from the index
    file's `weight_map` when present, else from the headers of every
    `*.safetensors` file in the directory (or of the one file given)."""

    def __init__(self, path: str | os.PathLike):
        from safetensors import safe_open

        self._safe_open = safe_open
        path = Path(path)
        self._files: dict[str, Path] = {}
        self._open: dict[Path, object] = {}
        if path.is_file():
            self.root = path.parent
            for name in self._handle(path).keys():
                self._files[name] = path
        elif (path / INDEX_FILE).is_file():
            self.root = path
            with open(path / INDEX_FILE) as f:
                weight_map = json.load(f)["weight_map"]
            self._files = {name: path / fname for name, fname in weight_map.items()}
        else:
            self.root = path
            shards = sorted(path.glob("*.safetensors"))
            if not shards:
                raise FileNotFoundError(f"no {INDEX_FILE} or *.safetensors under {path}")
            for shard in shards:
                for name in self._handle(shard).keys():
                    self._files[name] = shard

    def _handle(self, file: Path):
        h = self._open.get(file)
        if h is None:
            h = self._safe_open(str(file), framework="pt", device="cpu")
            self._open[file] = h
        return h

    def __contains__(self, name: str) -> bool:
        return name in self._files

    def get(self, name: str, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
        """The tensor `name` on the CPU, checked against the expected shape and dtype."""
        if name not in self._files:
            raise KeyError(f"checkpoint has no tensor {name}")
        t = self._handle(self._files[name]).get_tensor(name)
        if tuple(t.shape) != tuple(shape) or t.dtype != dtype:
            raise ValueError(f"{name}: expected {dtype} {list(shape)}, found {t.dtype} {list(t.shape)}")
        return t


@dataclass
class MoELayerWeights:
    """One layer's local experts in the forward's operand formats.

    Packed (`load_moe_layer(..., pack=True)`): `w13` / `w2` are the int32
    packed operand buffers of ops.pack_w13 / ops.pack_w2 on the device.
    Unpacked (`pack=False`): `w13` / `w2` are e4m3 `[E, 4096, 7168]` /
    `[E, 7168, 2048]` CPU tensors in the reference's `gemm1_weights` /
    `gemm2_weights` layout (the reference's own `run_custom` packs them).
    """

    layer: int
    local_expert_offset: int
    w13: torch.Tensor
    w13_scale: torch.Tensor      # f32 [E, 32, 56]
    w2: torch.Tensor
    w2_scale: torch.Tensor       # f32 [E, 56, 16]
    routing_bias: torch.Tensor   # f32 [256]
    router_weight: torch.Tensor | None  # bf16 [256, 7168], if the checkpoint holds it
    packed: bool


def _expert_tensors(ck: Checkpoint, layer: int, e: int):
    f8 = torch.float8_e4m3fn
    up = ck.get(expert_key(layer, e, "up_proj"), (I_DIM, H), f8)
    gate = ck.get(expert_key(layer, e, "gate_proj"), (I_DIM, H), f8)
    down = ck.get(expert_key(layer, e, "down_proj"), (H, I_DIM), f8)
    up_s = ck.get(expert_key(layer, e, "up_proj", "weight_scale_inv"), (I_BLOCKS, H_BLOCKS), torch.float32)
    gate_s = ck.get(expert_key(layer, e, "gate_proj", "weight_scale_inv"), (I_BLOCKS, H_BLOCKS), torch.float32)
    down_s = ck.get(expert_key(layer, e, "down_proj", "weight_scale_inv"), (H_BLOCKS, I_BLOCKS), torch.float32)
    return up, gate, down, up_s, gate_s, down_s


def load_moe_layer(path: str | os.PathLike, layer: int, local_expert_offset: int = 0, n_local: int = MAX_E_LOCAL,
                   device: str | torch.device = "cuda", pack: bool = True) -> MoELayerWeights:
    """Read experts local_expert_offset .. +n_local of `layer`.

    pack=True writes every expert straight into the packed operand buffers on
    `device` (a HIP device: packing runs the library's pack kernels, and a
    missing library raises).  pack=False returns the unpacked reference
    layout on the CPU.
    """
    if not (0 < n_local <= MAX_E_LOCAL):
        raise ValueError(f"n_local must be in 1..{MAX_E_LOCAL}")
    if local_expert_offset < 0 or local_expert_offset + n_local > E_GLOBAL:
        raise ValueError(f"experts {local_expert_offset}..{local_expert_offset + n_local - 1} are not all in 0..255")
    ck = Checkpoint(path)
    w13_scale = torch.empty((n_local, G1_BLOCKS, H_BLOCKS), dtype=torch.float32)
    w2_scale = torch.empty((n_local, H_BLOCKS, I_BLOCKS), dtype=torch.float32)
    routing_bias = ck.get(bias_key(layer), (E_GLOBAL,), torch.float32).clone()
    router = ck.get(router_key(layer), (E_GLOBAL, H), torch.bfloat16).clone() if router_key(layer) in ck else None

    if pack:
        from . import ops

        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("pack=True needs a HIP device (the packs run on the GPU)")
        w13 = torch.empty((n_local, *W13_PACKED_SHAPE), dtype=torch.int32, device=dev)
        w2 = torch.empty((n_local, *W2_PACKED_SHAPE), dtype=torch.int32, device=dev)
        stage13 = torch.empty((1, 2 * I_DIM, H), dtype=torch.float8_e4m3fn, device=dev)
        stage2 = torch.empty((1, H, I_DIM), dtype=torch.float8_e4m3fn, device=dev)
    else:
        w13 = torch.empty((n_local, 2 * I_DIM, H), dtype=torch.float8_e4m3fn)
        w2 = torch.empty((n_local, H, I_DIM), dtype=torch.float8_e4m3fn)

    for le in range(n_local):
        up, gate, down, up_s, gate_s, down_s = _expert_tensors(ck, layer, local_expert_offset + le)
        w13_scale[le, :I_BLOCKS] = up_s
        w13_scale[le, I_BLOCKS:] = gate_s
        w2_scale[le] = down_s
        if pack:
            # The staging copies are ordered on the current stream before the
            # packs that read them, and each copy waits for the previous pack.
            stage13[0, :I_DIM].copy_(up)
            stage13[0, I_DIM:].copy_(gate)
            stage2[0].copy_(down)
            ops.pack_w13(stage13, out=w13[le:le + 1])
            ops.pack_w2(stage2, out=w2[le:le + 1])
        else:
            w13[le, :I_DIM] = up
            w13[le, I_DIM:] = gate
            w2[le] = down

    if pack:
        w13_scale, w2_scale = w13_scale.to(dev), w2_scale.to(dev)
        routing_bias = routing_bias.to(dev)
        router = router.to(dev) if router is not None else None
        torch.cuda.current_stream(dev).synchronize()
    return MoELayerWeights(layer, local_expert_offset, w13, w13_scale, w2, w2_scale, routing_bias, router, pack)


def save_moe_layer(path: str | os.PathLike, layer: int, experts: dict, routing_bias: torch.Tensor,
                   router_weight: torch.Tensor | None = None, shards: int = 1) -> None:
    """Write expert tensors in the checkpoint layout (for tests and for
    converting other sources).  `experts` maps a global expert id to
    (gemm1_weights [4096, 7168], gemm1_weights_scale [32, 56],
    gemm2_weights [7168, 2048], gemm2_weights_scale [56, 16]) in the
    forward's layout; rows [0, 2048) of GEMM1 are written as up_proj and rows
    [2048, 4096) as gate_proj, the inverse of `load_moe_layer`.  With
    shards > 1 the tensors are spread over several files with an index."""
    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    tensors = {bias_key(layer): routing_bias.to(torch.float32).contiguous().cpu()}
    if router_weight is not None:
        tensors[router_key(layer)] = router_weight.to(torch.bfloat16).contiguous().cpu()
    for e, (w13, s13, w2, s2) in experts.items():
        w13, s13, w2, s2 = (t.contiguous().cpu() for t in (w13, s13, w2, s2))
        tensors[expert_key(layer, e, "up_proj")] = w13[:I_DIM].contiguous()
        tensors[expert_key(layer, e, "gate_proj")] = w13[I_DIM:].contiguous()
        tensors[expert_key(layer, e, "up_proj", "weight_scale_inv")] = s13[:I_BLOCKS].to(torch.float32).contiguous()
        tensors[expert_key(layer, e, "gate_proj", "weight_scale_inv")] = s13[I_BLOCKS:].to(torch.float32).contiguous()
        tensors[expert_key(layer, e, "down_proj")] = w2
        tensors[expert_key(layer, e, "down_proj", "weight_scale_inv")] = s2.to(torch.float32).contiguous()
    names = sorted(tensors)
    if shards <= 1:
        save_file(tensors, str(path / "model.safetensors"))
        return
    weight_map = {}
    for k in range(shards):
        part = names[k::shards]
        fname = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
        save_file({n: tensors[n] for n in part}, str(path / fname))
        weight_map.update({n: fname for n in part})
    with open(path / INDEX_FILE, "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
