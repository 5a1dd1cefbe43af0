"""MI355X-native FP8 MoE forward for the DeepSeek-V3/R1 routed-expert layer.

Drop-in for the ``moe_forward`` path of the reference (kernels/moe.cu,
moe_layer.py): hand-written gfx950 HIP kernels behind a C ABI
(include/moe_fp8.h), called from Python through ctypes with PyTorch tensors
supplying device memory and streams.

The package directory name starts with a digit, so import it with
``importlib.import_module("15642_moe_amd")``.
"""

from . import geometry  # noqa: F401

__all__ = ["geometry", "ops", "moe_layer", "inputs", "capi", "checkpoint"]


def __getattr__(name):
    if name in ("ops", "moe_layer", "inputs", "capi", "checkpoint"):
        import importlib

        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
