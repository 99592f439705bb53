"""Two-stage Marlin MoE layer orchestration (reference
vllm/model_executor/layers/fused_moe/fused_marlin_moe.py:50-382 and
moe_align_block_size.py:8-34).

Stage 1: moe_wna16_marlin_gemm(x, w13) over expert-sorted route blocks (top_k routes per
token, no router weight); SiLU-gated activation silu(h[:, :I]) * h[:, I:]
(activation.py:45-52); stage 2: moe_wna16_marlin_gemm(act, w2) with top_k=1 and the router
weights fused into the epilogue; finally the top-k sum.
"""
from __future__ import annotations

import torch

from . import _custom_ops as ops
from .scalar_type import ScalarType, scalar_types


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                         expert_map: torch.Tensor | None = None,
                         ignore_invalid_experts: bool = False):
    """Allocates the aligned-routing tensors and fills them on the device
    (moe_align_block_size.py:8-34)."""
    max_num_tokens_padded = topk_ids.numel() + num_experts * (block_size - 1)
    sorted_ids = torch.empty((max_num_tokens_padded,), dtype=torch.int32, device=topk_ids.device)
    expert_ids = torch.empty((max_num_tokens_padded // block_size + 1,), dtype=torch.int32,
                             device=topk_ids.device)
    num_tokens_post_pad = torch.empty((1,), dtype=torch.int32, device=topk_ids.device)
    ops.moe_align_block_size(topk_ids, num_experts, block_size, sorted_ids, expert_ids,
                             num_tokens_post_pad, expert_map)
    return sorted_ids, expert_ids, num_tokens_post_pad


def select_block_size_m(m: int, topk: int, num_experts: int) -> int:
    """fused_marlin_moe.py:319-321."""
    for block_size_m in (8, 16, 32, 48, 64):
        if m * topk / num_experts / block_size_m < 0.9:
            break
    return block_size_m


def silu_and_mul(out: torch.Tensor, x: torch.Tensor) -> None:
    """out = silu(x[..., :d]) * x[..., d:] (activation.py:45-52) in one native pass."""
    from . import capi

    capi.silu_and_mul(out, x.contiguous())


def fused_marlin_moe(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                     bias1: torch.Tensor | None, bias2: torch.Tensor | None,
                     w1_scale: torch.Tensor, w2_scale: torch.Tensor,
                     topk_weights: torch.Tensor, topk_ids: torch.Tensor, quant_type_id: int,
                     apply_router_weight_on_input: bool = False, global_num_experts: int = -1,
                     expert_map: torch.Tensor | None = None,
                     global_scale1: torch.Tensor | None = None,
                     global_scale2: torch.Tensor | None = None,
                     w1_zeros: torch.Tensor | None = None, w2_zeros: torch.Tensor | None = None,
                     is_w1_zp_float: bool = False, is_w2_zp_float: bool = False,
                     workspace: torch.Tensor | None = None, output: torch.Tensor | None = None,
                     inplace: bool = False, block_size_m: int | None = None,
                     moe_sum=None) -> torch.Tensor:
    quant_type = ScalarType.from_id(quant_type_id)
    bit4 = (scalar_types.uint4, scalar_types.uint4b8, scalar_types.float4_e2m1f)
    num_bits = 4 if quant_type in bit4 else 8
    m, k = hidden_states.shape
    e = w1.shape[0]
    topk = topk_ids.shape[1]
    n = w2.shape[1] * 16  # intermediate size (w2 is [E, I/16, K*bits/2])
    assert w1.shape[1] * 16 == k, "Hidden size mismatch w1"
    assert w2.shape[2] // (num_bits // 2) == k, "Hidden size mismatch w2"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert hidden_states.dtype in (torch.float16, torch.bfloat16)
    assert topk_weights.dtype == torch.float32

    if block_size_m is None:
        block_size_m = select_block_size_m(m, topk, e)
    if global_num_experts == -1:
        global_num_experts = e
    sorted_token_ids, expert_ids, num_tokens_post_padded = moe_align_block_size(
        topk_ids, block_size_m, global_num_experts, expert_map)
    if workspace is None:
        workspace = torch.empty(0, dtype=torch.int, device=hidden_states.device)

    cache13 = torch.empty((m * topk * max(2 * n, k),), device=hidden_states.device,
                          dtype=hidden_states.dtype)
    cache1 = cache13[: m * topk * 2 * n].view(m * topk, 2 * n)
    cache3 = cache13[: m * topk * k].view(m * topk, k)
    cache2 = torch.empty((m * topk, n), device=hidden_states.device, dtype=hidden_states.dtype)

    cache1 = ops.moe_wna16_marlin_gemm(
        hidden_states, cache1, w1, bias1, w1_scale, None, global_scale1, w1_zeros, None, None,
        workspace, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
        moe_block_size=block_size_m, top_k=topk, mul_topk_weights=apply_router_weight_on_input,
        b_q_type=quant_type, size_m=m, size_n=2 * n, size_k=k, is_k_full=True,
        use_atomic_add=False, use_fp32_reduce=True, is_zp_float=is_w1_zp_float)
    silu_and_mul(cache2, cache1.view(-1, 2 * n))
    if expert_map is not None:
        cache3.zero_()
    out3 = ops.moe_wna16_marlin_gemm(
        cache2, cache3, w2, bias2, w2_scale, None, global_scale2, w2_zeros, None, None,
        workspace, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
        moe_block_size=block_size_m, top_k=1, mul_topk_weights=not apply_router_weight_on_input,
        b_q_type=quant_type, size_m=m * topk, size_n=k, size_k=n, is_k_full=True,
        use_atomic_add=False, use_fp32_reduce=True, is_zp_float=is_w2_zp_float).view(-1, topk, k)

    if output is None:
        output = hidden_states if inplace else torch.empty_like(hidden_states)
    if moe_sum is None:
        return torch.sum(out3, dim=1, out=output)
    return moe_sum(out3, output)
