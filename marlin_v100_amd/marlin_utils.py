"""Weight-metadata preprocessing and linear-apply helpers with the reference's names
(reference vllm/model_executor/layers/quantization/utils/marlin_utils.py and
marlin_utils_fp4.py).  These produce exactly the metadata formats the ops consume:
scales and float zero points in logical [G, N] order, biases in marlin_permute_bias order,
NVFP4 scales in S0E5M3 encoding, MXFP4 scales as raw e8m0.
"""
from __future__ import annotations

import torch

from . import _custom_ops as ops
from .scalar_type import ScalarType, scalar_types


def marlin_make_workspace_new(device: torch.device, max_blocks_per_sm: int = 1) -> torch.Tensor:
    """The ops own their split-K scratch, so the workspace is empty
    (marlin_utils.py:248-252)."""
    return torch.empty(0, dtype=torch.int, device=device)


def get_scale_perms() -> tuple[list[int], list[int]]:
    """marlin_utils.py:279-286."""
    scale_perm: list[int] = []
    for i in range(8):
        scale_perm.extend([i + 8 * j for j in range(8)])
    scale_perm_single: list[int] = []
    for i in range(4):
        scale_perm_single.extend([2 * i + j for j in [0, 1, 8, 9, 16, 17, 24, 25]])
    return scale_perm, scale_perm_single


def marlin_logical_scales(s: torch.Tensor, size_k: int, size_n: int, group_size: int,
                          is_a_8bit: bool = False) -> torch.Tensor:
    """Scales / float zero points in logical N-contiguous [G, N] order
    (marlin_utils.py:302-307)."""
    return s.reshape((-1, size_n)).contiguous()


sm70_marlin_logical_scales = marlin_logical_scales


def marlin_moe_logical_scales(s: torch.Tensor, size_k: int, size_n: int, group_size: int,
                              is_a_8bit: bool = False) -> torch.Tensor:
    """[E, G, N] (marlin_utils.py:339-344)."""
    return s.reshape((s.shape[0], -1, size_n)).contiguous()


sm70_marlin_moe_logical_scales = marlin_moe_logical_scales


def marlin_permute_bias(s: torch.Tensor) -> torch.Tensor:
    """marlin_utils.py:310-314."""
    origin_shape = s.shape
    _, scale_perm_single = get_scale_perms()
    s = s.reshape((-1, len(scale_perm_single)))[:, scale_perm_single]
    return s.reshape(*origin_shape).contiguous()


# ---- act-order and integer zero points -----------------------------------------------------

MARLIN_SUPPORTED_GROUP_SIZES = [-1, 32, 64, 128]


def marlin_is_k_full(act_order: bool, is_row_parallel: bool) -> bool:
    """marlin_utils.py:255-256."""
    return (not act_order) or (act_order and not is_row_parallel)


def marlin_repeat_scales_on_all_ranks(act_order: bool, group_size: int,
                                      is_row_parallel: bool) -> bool:
    """marlin_utils.py:259-265."""
    return act_order or (group_size == -1 and is_row_parallel)


def marlin_make_empty_g_idx(device: torch.device) -> torch.Tensor:
    """marlin_utils.py:268-271."""
    return torch.nn.Parameter(torch.empty(0, dtype=torch.int, device=device),
                              requires_grad=False)


def marlin_sort_g_idx(g_idx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(sorted g_idx, sort indices) (marlin_utils.py:274-276).  The sort indices are the
    `perm` of gptq_marlin_repack and marlin_gemm."""
    g_idx_sort_indices = torch.argsort(g_idx).to(torch.int)
    return g_idx[g_idx_sort_indices], g_idx_sort_indices


def pack_cols(q_w: torch.Tensor, num_bits: int, size_k: int, size_n: int) -> torch.Tensor:
    """Pack codes along N, 32/num_bits per int32, column n in bits
    [num_bits*(n % pack), ...) (quant_utils.py:66-78)."""
    pack_factor = 32 // num_bits
    q_w = q_w.to(torch.int64)
    packed = torch.zeros((size_k, size_n // pack_factor), dtype=torch.int64, device=q_w.device)
    for idx in range(pack_factor):
        packed |= q_w[:, idx::pack_factor] << (num_bits * idx)
    return packed.to(torch.int32).contiguous()


def unpack_cols(q_w: torch.Tensor, num_bits: int, size_k: int, size_n: int) -> torch.Tensor:
    """Inverse of pack_cols (quant_utils.py:81-92)."""
    pack_factor = 32 // num_bits
    mask = (1 << num_bits) - 1
    unpacked = torch.empty((size_k, size_n), dtype=torch.int32, device=q_w.device)
    words = q_w.to(torch.int64)
    for idx in range(pack_factor):
        unpacked[:, idx::pack_factor] = ((words >> (num_bits * idx)) & mask).to(torch.int32)
    return unpacked.contiguous()


def marlin_zero_points(zp: torch.Tensor, size_k: int, size_n: int, num_bits: int,
                       is_a_8bit: bool = False) -> torch.Tensor:
    """Integer zero points [G, N] -> the packed int32 [G, N/pack] the ops take with
    is_zp_float=False.  The reference (marlin_utils.py:347-368) permutes and interleaves them
    for its SM80 fragment layout; the gfx950 kernels read metadata in logical column order,
    so this build packs them plainly along N (pack_cols)."""
    if num_bits not in (4, 8):
        raise ValueError(f"num_bits must be 4 or 8, got {num_bits}")
    return pack_cols(zp.reshape(-1, size_n), num_bits, zp.numel() // size_n, size_n)


def _awq_zp_logical(q_zp_packed: torch.Tensor, size_k: int, size_n: int,
                    num_bits: int) -> torch.Tensor:
    """AWQ packed zero points [G, N/pack] (codes interleaved [0,2,4,6,1,3,5,7] / [0,2,1,3]
    within each word) -> integer codes [G, N] (marlin_utils.py:382-393)."""
    q_zp = unpack_cols(q_zp_packed, num_bits, size_k, size_n)
    interleave = [0, 2, 4, 6, 1, 3, 5, 7] if num_bits == 4 else [0, 2, 1, 3]
    undo = torch.argsort(torch.tensor(interleave))
    return q_zp.reshape((-1, len(interleave)))[:, undo].reshape((-1, size_n)).contiguous()


def awq_to_marlin_zero_points(q_zp_packed: torch.Tensor, size_k: int, size_n: int,
                              num_bits: int, is_a_8bit: bool = False) -> torch.Tensor:
    """AWQ packed zero points -> this build's packed int32 zero points
    (marlin_utils.py:371-396)."""
    return marlin_zero_points(_awq_zp_logical(q_zp_packed, size_k, size_n, num_bits), size_k,
                              size_n, num_bits, is_a_8bit)


def awq_to_marlin_zero_points_float(q_zp_packed: torch.Tensor, scales: torch.Tensor, size_k: int,
                                    size_n: int, num_bits: int, scale_size_k: int,
                                    group_size: int, is_a_8bit: bool = False) -> torch.Tensor:
    """AWQ packed zero points -> float zero points dtype(z * s) in logical [G, N] order
    (marlin_utils.py:399-458)."""
    q_zp = _awq_zp_logical(q_zp_packed, size_k, size_n, num_bits)
    zp_float = (q_zp.float() * scales.contiguous().float()).to(scales.dtype)
    return marlin_logical_scales(zp_float, scale_size_k, size_n, group_size, is_a_8bit)


awq_to_sm70_marlin_zero_points_float = awq_to_marlin_zero_points_float


def moe_awq_to_marlin_zero_points(q_zp_packed: torch.Tensor, size_k: int, size_n: int,
                                  num_bits: int, is_a_8bit: bool = False) -> torch.Tensor:
    """Per-expert awq_to_marlin_zero_points (marlin_utils.py:461-478)."""
    return torch.stack([awq_to_marlin_zero_points(q_zp_packed[e], size_k, size_n, num_bits,
                                                  is_a_8bit)
                        for e in range(q_zp_packed.shape[0])])


def moe_awq_to_marlin_zero_points_float(q_zp_packed: torch.Tensor, scales: torch.Tensor,
                                        size_k: int, size_n: int, num_bits: int,
                                        scale_size_k: int, group_size: int,
                                        is_a_8bit: bool = False) -> torch.Tensor:
    """Per-expert awq_to_marlin_zero_points_float (marlin_utils.py:481-508)."""
    return torch.stack([awq_to_marlin_zero_points_float(q_zp_packed[e], scales[e], size_k,
                                                        size_n, num_bits, scale_size_k,
                                                        group_size, is_a_8bit)
                        for e in range(q_zp_packed.shape[0])])


def marlin_zero_points_float(zeros_int: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Integer zero points z [G, N] -> float zero points dtype(z * s) as the kernel takes them
    (marlin_utils.py:430-458, 511-538; tests/helpers.py:1249)."""
    return (zeros_int.to(torch.float32) * scales.to(torch.float32)).to(scales.dtype).contiguous()


# ---- FP4 ----------------------------------------------------------------------------------

def _nvfp4_compute_scale_factor(marlin_scales: torch.Tensor,
                                a_dtype: torch.dtype | None = None) -> float:
    """marlin_utils_fp4.py:30-50."""
    if a_dtype is not None and a_dtype == torch.half:
        return 1.0
    ws_float = marlin_scales.float() * (2 ** 7)
    nonzero_mask = ws_float > 0
    if nonzero_mask.any():
        min_val = ws_float[nonzero_mask].min()
        if min_val < 2:
            return float((2 / min_val).log2().ceil().exp2().item())
    return 1.0


def nvfp4_marlin_process_scales(marlin_scales: torch.Tensor, scale_factor: float | None = None,
                                a_dtype: torch.dtype | None = None):
    """e4m3 scales [G, N] -> S0E5M3 bytes, [0,2,1,3]-shuffled per 4 columns
    (marlin_utils_fp4.py:53-110)."""
    marlin_scales = marlin_scales.to(torch.half)
    marlin_scales = marlin_scales.view(-1, 4)[:, [0, 2, 1, 3]].view(marlin_scales.size(0), -1)
    if scale_factor is None:
        scale_factor = _nvfp4_compute_scale_factor(marlin_scales, a_dtype)
    if scale_factor > 1.0:
        marlin_scales = (marlin_scales.float() * scale_factor).to(torch.half)
    marlin_scales = (marlin_scales * (2 ** 7)).view(torch.int16) << 1
    marlin_scales = marlin_scales.view(torch.float8_e4m3fn)
    marlin_scales = marlin_scales[:, 1::2].contiguous()
    return marlin_scales, scale_factor


def nvfp4_marlin_process_global_scale(global_scale: torch.Tensor,
                                      a_dtype: torch.dtype | None = None) -> torch.Tensor:
    """marlin_utils_fp4.py:132-144."""
    if a_dtype is None:
        a_dtype = global_scale.dtype
    assert a_dtype in (torch.half, torch.bfloat16)
    target_exponent = 5 if a_dtype == torch.half else 8
    exponent_bias = 2 ** (target_exponent - 1) - 2 ** (2 - 1)
    return global_scale * (2.0 ** (exponent_bias - 7))


def mxfp4_marlin_process_scales(marlin_scales: torch.Tensor,
                                input_dtype: torch.dtype | None = None) -> torch.Tensor:
    """MXFP4 scales as raw e8m0 in logical [G, N] order, the order the kernels read
    (reference kernel sm70_marlin_mxfp4_gemm.cu:63-77 and tests/helpers.py:1081-1087).  The
    reference's vLLM helper additionally shuffles [0,2,1,3] for 16-bit activations
    (marlin_utils_fp4.py:115-129), which its own kernel does not undo; this build keeps the
    kernel's logical order."""
    if input_dtype is not None and input_dtype.itemsize == 1:
        raise RuntimeError("8-bit activations are not supported on this build")
    return marlin_scales.to(torch.float8_e8m0fnu).contiguous()


# ---- linear apply ------------------------------------------------------------------------

def apply_gptq_marlin_linear(input: torch.Tensor, weight: torch.Tensor,
                             weight_scale: torch.Tensor, weight_zp: torch.Tensor | None,
                             g_idx: torch.Tensor | None, g_idx_sort_indices: torch.Tensor | None,
                             workspace: torch.Tensor, wtype: ScalarType,
                             output_size_per_partition: int, input_size_per_partition: int,
                             is_k_full: bool = True,
                             input_global_scale: torch.Tensor | None = None,
                             bias: torch.Tensor | None = None, use_fp32_reduce: bool = True,
                             input_dtype: torch.dtype | None = None,
                             is_zp_float: bool = False) -> torch.Tensor:
    """marlin_utils.py:631-696 (bias already in marlin_permute_bias order).  Zero points are
    float ([G, N], is_zp_float=True) or packed int32 ([G, N/pack]); act-order passes the
    sorted g_idx and its sort indices."""
    if input_dtype is not None and input_dtype.itemsize == 1:
        raise RuntimeError("8-bit activations are not supported on this build")
    reshaped_x = input.reshape(-1, input.shape[-1])
    out_shape = input.shape[:-1] + (output_size_per_partition,)
    has_zp = weight_zp is not None and weight_zp.numel() > 0
    output = ops.marlin_gemm(reshaped_x, None, weight, bias, weight_scale, None, None,
                             weight_zp if has_zp else None, g_idx, g_idx_sort_indices, workspace,
                             wtype, size_m=reshaped_x.shape[0],
                             size_n=output_size_per_partition, size_k=input_size_per_partition,
                             is_k_full=is_k_full, use_atomic_add=False,
                             use_fp32_reduce=use_fp32_reduce,
                             is_zp_float=has_zp and is_zp_float)
    return output.reshape(out_shape)


def apply_awq_marlin_linear(input: torch.Tensor, weight: torch.Tensor,
                            weight_scale: torch.Tensor, weight_zp: torch.Tensor,
                            g_idx: torch.Tensor | None, g_idx_sort_indices: torch.Tensor | None,
                            workspace: torch.Tensor, quant_type: ScalarType,
                            output_size_per_partition: int, input_size_per_partition: int,
                            bias: torch.Tensor | None = None,
                            use_fp32_reduce: bool = True) -> torch.Tensor:
    """marlin_utils.py:699-761 with float zero points (is_zp_float=True)."""
    reshaped_x = input.reshape(-1, input.shape[-1])
    out_shape = input.shape[:-1] + (output_size_per_partition,)
    output = ops.marlin_gemm(reshaped_x, None, weight, bias, weight_scale, None, None, weight_zp,
                             g_idx, g_idx_sort_indices, workspace, quant_type,
                             size_m=reshaped_x.shape[0], size_n=output_size_per_partition,
                             size_k=input_size_per_partition, use_atomic_add=False,
                             use_fp32_reduce=use_fp32_reduce, is_zp_float=True)
    return output.reshape(out_shape)


def apply_fp4_marlin_linear(input: torch.Tensor, weight: torch.Tensor,
                            weight_scale: torch.Tensor, weight_global_scale: torch.Tensor | None,
                            workspace: torch.Tensor, size_n: int, size_k: int,
                            bias: torch.Tensor | None = None,
                            input_dtype: torch.dtype | None = None,
                            use_fp32_reduce: bool = True) -> torch.Tensor:
    """marlin_utils_fp4.py:147-201 (16-bit activations only)."""
    if input_dtype is not None and input_dtype.itemsize == 1:
        raise RuntimeError("8-bit activations are not supported on this build")
    reshaped_x = input.reshape(-1, input.shape[-1])
    out_shape = input.shape[:-1] + (size_n,)
    output = ops.marlin_gemm(reshaped_x, None, weight, bias, weight_scale, None,
                             weight_global_scale, None, None, None, workspace,
                             scalar_types.float4_e2m1f, size_m=reshaped_x.shape[0], size_n=size_n,
                             size_k=size_k, use_atomic_add=False,
                             use_fp32_reduce=use_fp32_reduce, is_zp_float=False)
    return output.reshape(out_shape)
