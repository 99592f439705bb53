"""Two-stage Marlin MoE layer orchestration (reference
vllm/model_executor/layers/fused_moe/fused_marlin_moe.py:50-382 and
moe_align_block_size.py:8-34).

Stage 1: moe_wna16_marlin_gemm(x, w13) over expert-sorted route blocks (top_k routes per
token, no router weight); the gated activation, silu(h[:, :I]) * h[:, I:] by default
(activation.py:45-52); stage 2: moe_wna16_marlin_gemm(act, w2) with top_k=1 and the router
weights fused into the epilogue; finally the top-k sum.

`fused_marlin_moe` keeps the reference's parameter names, order and defaults, so keyword
and positional callers work unchanged.  The SiLU-gated activation with the default
activation callback runs as one native pass; any other activation goes through
`activation_func` (torch on the device, as in the reference).  Act-order tensors
(g_idx / sort_indices) and 8-bit activations (input_dtype int8 / fp8) raise
NotImplementedError: the GEMM op rejects them, as the reference's does (marlin.cu:95-102).
"""
from __future__ import annotations

from collections.abc import Callable
from enum import Enum

import torch
import torch.nn.functional as F

from . import _custom_ops as ops
from .scalar_type import ScalarType, scalar_types


class MoEActivation(Enum):
    """Activation names of the reference (activation.py:9-37)."""
    SILU = "silu"
    GELU = "gelu"
    RELU2 = "relu2"
    SWIGLUOAI = "swigluoai"
    SWIGLUSTEP = "swiglustep"
    SILU_NO_MUL = "silu_no_mul"
    GELU_NO_MUL = "gelu_no_mul"
    RELU2_NO_MUL = "relu2_no_mul"

    @property
    def is_gated(self) -> bool:
        return not self.value.endswith("_no_mul")

    @classmethod
    def from_str(cls, value: str) -> "MoEActivation":
        for act in cls:
            if act.value == value:
                return act
        raise ValueError(f"Unknown MoE activation: {value!r}")


def apply_moe_activation(activation: MoEActivation, output: torch.Tensor,
                         input: torch.Tensor) -> torch.Tensor:
    """The reference's activation callback (activation.py:45-72), in torch on the device."""
    if activation == MoEActivation.SILU:
        gate, up = input.chunk(2, dim=-1)
        output.copy_(F.silu(gate) * up)
    elif activation == MoEActivation.GELU:
        gate, up = input.chunk(2, dim=-1)
        output.copy_(F.gelu(gate) * up)
    elif activation == MoEActivation.RELU2:
        gate, up = input.chunk(2, dim=-1)
        output.copy_(F.relu(gate).square() * up)
    elif activation == MoEActivation.SILU_NO_MUL:
        output.copy_(F.silu(input))
    elif activation == MoEActivation.GELU_NO_MUL:
        output.copy_(F.gelu(input))
    elif activation == MoEActivation.RELU2_NO_MUL:
        output.copy_(F.relu(input).square())
    else:
        raise NotImplementedError(f"Unsupported MoE activation: {activation}")
    return output


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                         expert_map: torch.Tensor | None = None,
                         ignore_invalid_experts: bool = False):
    """Allocates the aligned-routing tensors and fills them on the device
    (moe_align_block_size.py:8-34).  Invalid ids are always skipped."""
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


def _stage1_silu_fused(x, out, w1, bias1, w1_scale, global_scale1, w1_zeros, sorted_token_ids,
                       expert_ids, num_tokens_post_padded, topk_weights, block_size_m, topk,
                       mul_topk, quant_type, size_m, size_n, size_k, is_zp_float) -> bool:
    """Stage 1 with the gated SiLU fused (marlin_moe_wna16_marlin_gemm_silu).  False when the
    library's plan for this batch cannot fuse it (nothing was launched then)."""
    from . import capi

    try:
        capi.moe_wna16_marlin_gemm(
            x, w1, w1_scale, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
            block_size_m, topk, mul_topk, quant_type.id, size_m, size_n, size_k, c=out,
            b_bias=bias1, global_scale=global_scale1, b_zeros=w1_zeros,
            is_zp_float=is_zp_float, silu_gated=True)
    except capi.MarlinError as err:
        if err.status == capi.STATUS_NOT_SUPPORTED:
            return False
        raise
    return True


def _unsupported(name: str, t) -> bool:
    return t is not None and (not isinstance(t, torch.Tensor) or t.numel() > 0)


def fused_marlin_moe(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                     bias1: torch.Tensor | None, bias2: torch.Tensor | None,
                     w1_scale: torch.Tensor, w2_scale: torch.Tensor,
                     topk_weights: torch.Tensor, topk_ids: torch.Tensor, quant_type_id: int,
                     apply_router_weight_on_input: bool = False, global_num_experts: int = -1,
                     activation: MoEActivation = MoEActivation.SILU,
                     activation_func: Callable[[MoEActivation, torch.Tensor, torch.Tensor],
                                               None] = apply_moe_activation,
                     moe_sum: Callable[[torch.Tensor, torch.Tensor], None] | None = None,
                     expert_map: torch.Tensor | None = None,
                     input_global_scale1: torch.Tensor | None = None,
                     input_global_scale2: torch.Tensor | None = None,
                     global_scale1: torch.Tensor | None = None,
                     global_scale2: torch.Tensor | None = None,
                     g_idx1: torch.Tensor | None = None, g_idx2: torch.Tensor | None = None,
                     sort_indices1: torch.Tensor | None = None,
                     sort_indices2: torch.Tensor | None = None,
                     w1_zeros: torch.Tensor | None = None, w2_zeros: torch.Tensor | None = None,
                     is_w1_zp_float: bool = False, is_w2_zp_float: bool = False,
                     workspace: torch.Tensor | None = None,
                     intermediate_cache13: torch.Tensor | None = None,
                     intermediate_cache2: torch.Tensor | None = None,
                     is_k_full: bool = True, output: torch.Tensor | None = None,
                     input_dtype: torch.dtype | None = None, inplace: bool = False, *,
                     block_size_m: int | None = None,
                     fuse_activation: bool = False) -> torch.Tensor:
    """The reference's fused_marlin_moe (fused_marlin_moe.py:217-382).  Keyword-only
    extensions (not in the reference): `block_size_m` fixes the moe block size instead of the
    reference's heuristic; `fuse_activation` runs stage 1 with the SiLU-gated activation in
    its epilogue where the library's plan allows it (same bits as the two passes).  It is off
    by default: on the BASELINE cfg5 shape the fused stage-1 kernels measured slower than
    stage 1 plus the activation pass, at T = 2048 (661 against 608 + 29 us per kernel) and
    for decode-sized batches (T = 16 / 32 / 64 layer: 161 / 246 / 342 against 142 / 214 /
    299 us), where each wave streams two 2 KiB pieces N/2 apart instead of 4 KiB."""
    if inplace:
        assert output is None, "Conflicting request"
    if isinstance(activation, str):
        activation = MoEActivation.from_str(activation)
    for name, t in (("g_idx1", g_idx1), ("g_idx2", g_idx2), ("sort_indices1", sort_indices1),
                    ("sort_indices2", sort_indices2)):
        if _unsupported(name, t):
            raise NotImplementedError(f"{name}: act-order is not supported by "
                                      "moe_wna16_marlin_gemm (as in the reference)")
    if input_dtype is not None and input_dtype.itemsize == 1:
        raise NotImplementedError("8-bit activations (input_dtype int8 / fp8) are not supported")
    if input_global_scale1 is not None or input_global_scale2 is not None:
        raise NotImplementedError("input_global_scale applies to 8-bit activations only")

    quant_type = ScalarType.from_id(quant_type_id)
    assert quant_type in (scalar_types.uint4, scalar_types.uint8, scalar_types.uint8b128,
                          scalar_types.uint4b8, scalar_types.float8_e4m3fn,
                          scalar_types.float4_e2m1f)
    bit4 = (scalar_types.uint4, scalar_types.uint4b8, scalar_types.float4_e2m1f)
    num_bits = 4 if quant_type in bit4 else 8
    m, k = hidden_states.shape
    e = w1.shape[0]
    topk = topk_ids.shape[1]
    assert w1.shape[1] * 16 == k, "Hidden size mismatch w1"
    assert w2.shape[2] // (num_bits // 2) == k, "Hidden size mismatch w2"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert w2.is_contiguous(), "Expert weights2 must be contiguous"
    assert hidden_states.dtype in (torch.float16, torch.bfloat16)
    assert topk_weights.dtype == torch.float32
    n = w2.shape[1] * 16  # intermediate size (w2 is [E, I/16, K*bits/2])
    shards = 2 if activation.is_gated else 1

    if block_size_m is None:
        block_size_m = select_block_size_m(m, topk, e)
    if global_num_experts == -1:
        global_num_experts = e
    sorted_token_ids, expert_ids, num_tokens_post_padded = moe_align_block_size(
        topk_ids, block_size_m, global_num_experts, expert_map, ignore_invalid_experts=True)
    if workspace is None:
        workspace = torch.empty(0, dtype=torch.int, device=hidden_states.device)

    dev, dt = hidden_states.device, hidden_states.dtype
    if intermediate_cache13 is None:
        intermediate_cache13 = torch.empty((m * topk * max(shards * n, k),), device=dev, dtype=dt)
    if intermediate_cache2 is None:
        intermediate_cache2 = torch.empty((m * topk, n), device=dev, dtype=dt)
    cache1 = intermediate_cache13.flatten()[: m * topk * shards * n].view(m * topk, shards * n)
    cache3 = intermediate_cache13.flatten()[: m * topk * k].view(m * topk, k)
    cache2 = intermediate_cache2.flatten()[: m * topk * n].view(m * topk, n)

    default_silu = activation == MoEActivation.SILU and activation_func is apply_moe_activation
    fused = False
    if fuse_activation and default_silu:
        # stage 1 with silu(gate) * up in its epilogue: cache2 directly, no [T*topk, 2I]
        # intermediate and no activation pass (same bits as the two passes below)
        fused = _stage1_silu_fused(hidden_states, cache2, w1, bias1, w1_scale, global_scale1,
                                   w1_zeros, sorted_token_ids, expert_ids, num_tokens_post_padded,
                                   topk_weights, block_size_m, topk, apply_router_weight_on_input,
                                   quant_type, m, 2 * n, k, is_w1_zp_float)
    if not fused:
        cache1 = ops.moe_wna16_marlin_gemm(
            hidden_states, cache1, w1, bias1, w1_scale, None, global_scale1, w1_zeros, None,
            None, workspace, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
            moe_block_size=block_size_m, top_k=topk,
            mul_topk_weights=apply_router_weight_on_input, b_q_type=quant_type, size_m=m,
            size_n=shards * n, size_k=k, is_k_full=is_k_full, use_atomic_add=False,
            use_fp32_reduce=True, is_zp_float=is_w1_zp_float)
        if default_silu:
            silu_and_mul(cache2, cache1.view(-1, 2 * n))
        else:
            activation_func(activation, cache2, cache1.view(-1, shards * n))
    if expert_map is not None:
        cache3.zero_()
    out3 = ops.moe_wna16_marlin_gemm(
        cache2, cache3, w2, bias2, w2_scale, None, global_scale2, w2_zeros, None, None,
        workspace, sorted_token_ids, expert_ids, num_tokens_post_padded, topk_weights,
        moe_block_size=block_size_m, top_k=1, mul_topk_weights=not apply_router_weight_on_input,
        b_q_type=quant_type, size_m=m * topk, size_n=k, size_k=n, is_k_full=is_k_full,
        use_atomic_add=False, use_fp32_reduce=True, is_zp_float=is_w2_zp_float).view(-1, topk, k)

    if output is None:
        output = hidden_states if inplace else torch.empty_like(hidden_states)
    if moe_sum is None:
        return torch.sum(out3, dim=1, out=output)
    return moe_sum(out3, output)
