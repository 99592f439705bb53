"""MI355X (gfx950) Marlin mixed-precision GEMM behind the reference's torch op API.

`from marlin_v100_amd import ops` (or importing any op module) loads the two op libraries,
which register torch.ops._C.{marlin_gemm, gptq_marlin_repack, awq_marlin_repack} and
torch.ops._moe_C.{moe_align_block_size, moe_wna16_marlin_gemm, moe_sum}.  There is no
fallback: if the built extensions are missing, loading fails with ImportError.
"""
from __future__ import annotations

import importlib
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
_LOADED = False


def load_extensions() -> None:
    global _LOADED
    if _LOADED:
        return
    missing = [n for n in ("libmarlin_mi355x.so", "_C.so", "_moe_C.so")
               if not os.path.exists(os.path.join(_HERE, n))]
    if missing:
        raise ImportError(
            f"marlin_v100_amd native libraries not built ({', '.join(missing)}); run "
            "`python -m marlin_v100_amd.build` (or __graft_entry__.build())")
    import torch  # noqa: F401  (torch's HIP runtime must be loaded before our libraries)

    importlib.import_module(f"{__name__}._C")
    importlib.import_module(f"{__name__}._moe_C")
    _LOADED = True


def __getattr__(name):
    if name == "ops":
        return importlib.import_module(f"{__name__}._custom_ops")
    if name in ("ScalarType", "scalar_types"):
        return getattr(importlib.import_module(f"{__name__}.scalar_type"), name)
    raise AttributeError(name)
