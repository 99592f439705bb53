"""Builds quantized test cases with the oracle: logical weights, the packed source format a
caller hands to the repack ops, the metadata tensors the GEMM takes, and the oracle's
dequantized weights."""
from __future__ import annotations

from dataclasses import dataclass

import torch

import oracle as O

FORMATS = ("u4b8", "u4", "u8b128", "u8", "fp8", "mxfp4", "nvfp4")
TYPE_ID = {
    "u4b8": O.scalar_types.uint4b8.id,
    "u4": O.scalar_types.uint4.id,
    "u8b128": O.scalar_types.uint8b128.id,
    "u8": O.scalar_types.uint8.id,
    "fp8": O.scalar_types.float8_e4m3fn.id,
    "mxfp4": O.scalar_types.float4_e2m1f.id,
    "nvfp4": O.scalar_types.float4_e2m1f.id,
}
BITS = {"u4b8": 4, "u4": 4, "u8b128": 8, "u8": 8, "fp8": 8, "mxfp4": 4, "nvfp4": 4}
DEFAULT_GS = {"u4b8": 128, "u4": 128, "u8b128": -1, "u8": 128, "fp8": 128, "mxfp4": 32,
              "nvfp4": 16}


@dataclass
class QuantCase:
    fmt: str
    k: int
    n: int
    gs: int
    dtype: torch.dtype
    gptq_words: torch.Tensor        # [K/pack, N] int32 (GPTQ source for gptq_marlin_repack)
    awq_words: torch.Tensor | None  # [K, N/pack] int32 (integer formats only)
    scales: torch.Tensor            # kernel metadata [G, N]
    zeros: torch.Tensor | None      # float zero points [G, N] (u4 / u8)
    global_scale: torch.Tensor | None
    deq: torch.Tensor               # oracle dequantized weights [K, N] (dtype)
    gemm_alpha: float = 1.0         # the oracle GEMM uses deq directly

    @property
    def type_id(self) -> int:
        return TYPE_ID[self.fmt]


def make_case(fmt: str, k: int, n: int, dtype: torch.dtype, gs: int | None = None,
              seed: int = 0, std: float = 0.02) -> QuantCase:
    gen = torch.Generator().manual_seed(seed)
    gs = DEFAULT_GS[fmt] if gs is None else gs
    w = (torch.randn((k, n), generator=gen, dtype=torch.float32) * std).to(dtype)
    bits = BITS[fmt]
    awq = None
    zeros = None
    glob = None
    if fmt in ("u4b8", "u8b128"):
        q, s = O.quantize_with_bias(w, gs, 8 if fmt == "u4b8" else 128, dtype)
        deq = O.dequant_int(q, s, fmt, dtype)
        gptq = O.gptq_pack(q, bits)
        awq = O.awq_pack(q, bits)
        scales = s
    elif fmt in ("u4", "u8"):
        q, s, _z, zp = O.quantize_with_zero_point(w, gs, bits, dtype)
        deq = O.dequant_int(q, s, fmt, dtype, zp)
        gptq = O.gptq_pack(q, bits)
        awq = O.awq_pack(q, bits)
        scales, zeros = s, zp
    elif fmt == "fp8":
        fp8, s = O.quantize_fp8(w, gs, dtype)
        deq = O.dequant_fp8(fp8, s, dtype)
        raw = fp8.view(torch.uint8).to(torch.int32)
        gptq = O.gptq_pack(raw, 8)
        scales = s
    elif fmt == "mxfp4":
        q, s = O.quantize_mxfp4(w, 32)
        deq = O.dequant_mxfp4(q, s, dtype)
        gptq = O.fp4_to_gptq_words(q)
        scales = s
    elif fmt == "nvfp4":
        q, fp8s, g = O.quantize_nvfp4(w, 16)
        ps, sf = O.nvfp4_marlin_process_scales(fp8s, dtype)
        glob = (O.nvfp4_marlin_process_global_scale(g, dtype) / sf).to(torch.float32)
        deq = O.dequant_nvfp4(q, ps, glob, dtype)
        gptq = O.fp4_to_gptq_words(q)
        scales = ps
    else:
        raise ValueError(fmt)
    return QuantCase(fmt, k, n, gs, dtype, gptq, awq, scales, zeros, glob, deq)


def to_dev(case: QuantCase, device="cuda") -> QuantCase:
    def mv(t):
        return None if t is None else t.to(device)

    return QuantCase(case.fmt, case.k, case.n, case.gs, case.dtype, mv(case.gptq_words),
                     mv(case.awq_words), mv(case.scales), mv(case.zeros), mv(case.global_scale),
                     case.deq, case.gemm_alpha)
