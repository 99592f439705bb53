"""Python op wrappers with the reference's names and signatures
(reference vllm/_custom_ops.py:1163-1351, 2129-2168, 2286-2358, 2361-2483).

Each wrapper forwards to the torch op registered by _C.so / _moe_C.so, which validates the
arguments and calls the C ABI of libmarlin_mi355x.so.  Fake (meta) implementations let
torch.compile trace the ops.
"""
from __future__ import annotations

import torch

from . import load_extensions
from .scalar_type import ScalarType

load_extensions()

try:
    from torch.library import register_fake
except ImportError:  # older torch
    from torch.library import impl_abstract as register_fake


# ---- dense repack ------------------------------------------------------------------------

def gptq_marlin_repack(b_q_weight: torch.Tensor, perm: torch.Tensor, size_k: int, size_n: int,
                       num_bits: int, is_a_8bit: bool = False) -> torch.Tensor:
    return torch.ops._C.gptq_marlin_repack(b_q_weight, perm, size_k, size_n, num_bits, is_a_8bit)


@register_fake("_C::gptq_marlin_repack")
def _gptq_marlin_repack_fake(b_q_weight, perm, size_k, size_n, num_bits, is_a_8bit=False):
    pack_factor = 32 // num_bits
    return torch.empty((size_k // 16, size_n * 16 // pack_factor), dtype=b_q_weight.dtype,
                       device=b_q_weight.device)


def awq_marlin_repack(b_q_weight: torch.Tensor, size_k: int, size_n: int, num_bits: int,
                      is_a_8bit: bool = False) -> torch.Tensor:
    return torch.ops._C.awq_marlin_repack(b_q_weight, size_k, size_n, num_bits, is_a_8bit)


@register_fake("_C::awq_marlin_repack")
def _awq_marlin_repack_fake(b_q_weight, size_k, size_n, num_bits, is_a_8bit=False):
    pack_factor = 32 // num_bits
    return torch.empty((size_k // 16, size_n * 16 // pack_factor), dtype=b_q_weight.dtype,
                       device=b_q_weight.device)


def marlin_int4_fp8_preprocess(qweight: torch.Tensor, qzeros_or_none: torch.Tensor | None = None,
                               inplace: bool = False) -> torch.Tensor:
    """W4A8-FP8 code remap (reference marlin_int4_fp8_preprocess.cu:58-97)."""
    return torch.ops._C.marlin_int4_fp8_preprocess(qweight, qzeros_or_none, inplace)


@register_fake("_C::marlin_int4_fp8_preprocess")
def _marlin_int4_fp8_preprocess_fake(qweight, qzeros_or_none=None, inplace=False):
    return qweight if inplace else torch.empty_like(qweight)


def gptq_marlin_moe_repack(b_q_weight: torch.Tensor, perm: torch.Tensor, size_k: int,
                           size_n: int, num_bits: int, is_a_8bit: bool = False) -> torch.Tensor:
    """Per-expert repack into [E, size_k/16, size_n*bits/2] (reference _custom_ops.py:1228-1248)."""
    num_experts = b_q_weight.shape[0]
    assert size_k % 16 == 0
    output = torch.empty((num_experts, size_k // 16, size_n * (num_bits // 2)),
                         device=b_q_weight.device, dtype=b_q_weight.dtype)
    for e in range(num_experts):
        output[e] = torch.ops._C.gptq_marlin_repack(b_q_weight[e], perm[e], size_k, size_n,
                                                    num_bits, is_a_8bit)
    return output


def awq_marlin_moe_repack(b_q_weight: torch.Tensor, perm: torch.Tensor, size_k: int,
                          size_n: int, num_bits: int, is_a_8bit: bool = False) -> torch.Tensor:
    """Per-expert AWQ repack (reference _custom_ops.py:1251-1269)."""
    num_experts = b_q_weight.shape[0]
    assert size_k % 16 == 0
    output = torch.empty((num_experts, size_k // 16, size_n * (num_bits // 2)),
                         device=b_q_weight.device, dtype=b_q_weight.dtype)
    for e in range(num_experts):
        output[e] = torch.ops._C.awq_marlin_repack(b_q_weight[e], size_k, size_n, num_bits,
                                                   is_a_8bit)
    return output


# ---- dense GEMM --------------------------------------------------------------------------

def marlin_gemm(a: torch.Tensor, c: torch.Tensor | None, b_q_weight: torch.Tensor,
                b_bias: torch.Tensor | None, b_scales: torch.Tensor,
                a_scales: torch.Tensor | None, global_scale: torch.Tensor | None,
                b_zeros: torch.Tensor | None, g_idx: torch.Tensor | None,
                perm: torch.Tensor | None, workspace: torch.Tensor, b_q_type: ScalarType,
                size_m: int, size_n: int, size_k: int, is_k_full: bool = True,
                use_atomic_add: bool = False, use_fp32_reduce: bool = False,
                is_zp_float: bool = False) -> torch.Tensor:
    return torch.ops._C.marlin_gemm(a, c, b_q_weight, b_bias, b_scales, a_scales, global_scale,
                                    b_zeros, g_idx, perm, workspace, b_q_type.id, size_m, size_n,
                                    size_k, is_k_full, use_atomic_add, use_fp32_reduce,
                                    is_zp_float)


@register_fake("_C::marlin_gemm")
def _marlin_gemm_fake(a, c, b_q_weight, b_bias, b_scales, a_scales, global_scale, b_zeros, g_idx,
                      perm, workspace, b_q_type_id, size_m, size_n, size_k, is_k_full=True,
                      use_atomic_add=False, use_fp32_reduce=False, is_zp_float=False):
    dtype = a.dtype
    if dtype not in (torch.half, torch.bfloat16):
        dtype = b_scales.dtype
    return torch.empty((size_m, size_n), device=a.device, dtype=dtype)


# ---- MoE ---------------------------------------------------------------------------------

def topk_softmax(topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                 token_expert_indices: torch.Tensor, gating_output: torch.Tensor,
                 renormalize: bool = False,
                 e_score_correction_bias: torch.Tensor | None = None) -> None:
    torch.ops._moe_C.topk_softmax(topk_weights, topk_ids, token_expert_indices, gating_output,
                                  renormalize, e_score_correction_bias)


def topk_sigmoid(topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                 token_expert_indices: torch.Tensor, gating_output: torch.Tensor,
                 renormalize: bool = False,
                 e_score_correction_bias: torch.Tensor | None = None) -> None:
    torch.ops._moe_C.topk_sigmoid(topk_weights, topk_ids, token_expert_indices, gating_output,
                                  renormalize, e_score_correction_bias)


def grouped_topk(scores: torch.Tensor, num_expert_group: int, topk_group: int, topk: int,
                 renormalize: bool, routed_scaling_factor: float, bias: torch.Tensor,
                 scoring_func: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    return torch.ops._moe_C.grouped_topk(scores, num_expert_group, topk_group, topk,
                                         renormalize, routed_scaling_factor, bias, scoring_func)


@register_fake("_moe_C::grouped_topk")
def _grouped_topk_fake(scores, n_group, topk_group, topk, renormalize, routed_scaling_factor,
                       bias, scoring_func):
    return (torch.empty((scores.shape[0], topk), dtype=torch.float32, device=scores.device),
            torch.empty((scores.shape[0], topk), dtype=torch.int32, device=scores.device))


def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                         sorted_token_ids: torch.Tensor, experts_ids: torch.Tensor,
                         num_tokens_post_pad: torch.Tensor,
                         expert_map: torch.Tensor | None = None) -> None:
    torch.ops._moe_C.moe_align_block_size(topk_ids, num_experts, block_size, sorted_token_ids,
                                          experts_ids, num_tokens_post_pad, expert_map)


def moe_sum(input: torch.Tensor, output: torch.Tensor) -> None:
    torch.ops._moe_C.moe_sum(input, output)


def moe_wna16_marlin_gemm(input: torch.Tensor, output: torch.Tensor | None,
                          b_qweight: torch.Tensor, b_bias: torch.Tensor | None,
                          b_scales: torch.Tensor, a_scales: torch.Tensor | None,
                          global_scale: torch.Tensor | None, b_qzeros: torch.Tensor | None,
                          g_idx: torch.Tensor | None, perm: torch.Tensor | None,
                          workspace: torch.Tensor, sorted_token_ids: torch.Tensor,
                          expert_ids: torch.Tensor, num_tokens_past_padded: torch.Tensor,
                          topk_weights: torch.Tensor, moe_block_size: int, top_k: int,
                          mul_topk_weights: bool, b_q_type: ScalarType, size_m: int,
                          size_n: int, size_k: int, is_k_full: bool, use_atomic_add: bool,
                          use_fp32_reduce: bool, is_zp_float: bool, thread_k: int = -1,
                          thread_n: int = -1, blocks_per_sm: int = -1) -> torch.Tensor:
    return torch.ops._moe_C.moe_wna16_marlin_gemm(
        input, output, b_qweight, b_bias, b_scales, a_scales, global_scale, b_qzeros, g_idx,
        perm, workspace, sorted_token_ids, expert_ids, num_tokens_past_padded, topk_weights,
        moe_block_size, top_k, mul_topk_weights, b_q_type.id, size_m, size_n, size_k, is_k_full,
        use_atomic_add, use_fp32_reduce, is_zp_float, thread_k, thread_n, blocks_per_sm)


@register_fake("_moe_C::moe_wna16_marlin_gemm")
def _moe_wna16_marlin_gemm_fake(input, output, b_qweight, b_bias, b_scales, a_scales,
                                global_scale, b_qzeros, g_idx, perm, workspace, sorted_token_ids,
                                expert_ids, num_tokens_past_padded, topk_weights, moe_block_size,
                                top_k, mul_topk_weights, b_q_type_id, size_m, size_n, size_k,
                                is_k_full, use_atomic_add, use_fp32_reduce, is_zp_float,
                                thread_k=-1, thread_n=-1, blocks_per_sm=-1):
    return torch.empty((size_m * top_k, size_n), dtype=input.dtype, device=input.device)


# ---- inspection ---------------------------------------------------------------------------

def marlin_dequantize(b_q_weight: torch.Tensor, b_scales: torch.Tensor,
                      b_zeros: torch.Tensor | None, global_scale: torch.Tensor | None,
                      b_q_type: ScalarType, size_k: int, size_n: int,
                      out_dtype: torch.dtype) -> torch.Tensor:
    """Dequantize repacked weights with the GEMM's device dequant routines ([K, N])."""
    return torch.ops._marlin_mi355x.dequantize(b_q_weight, b_scales, b_zeros, global_scale,
                                               b_q_type.id, size_k, size_n, out_dtype)
