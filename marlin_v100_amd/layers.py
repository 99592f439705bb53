"""Layer integration: the weight-loading and apply steps of the vLLM layer classes that sit
above the Marlin ops, for GPTQ / AWQ checkpoints on this build.

Mirrors (reference file:line):
  * MPLinearLayerConfig, MarlinLinearKernel.process_weights_after_loading / apply_weights
    (vllm/model_executor/kernels/linear/mixed_precision/MPLinearKernel.py:14-24,
    marlin.py:68-214);
  * the AWQ checkpoint conversion and AWQMarlinLinearMethod (awq_marlin.py:75-130, 355-483);
  * AWQMarlinMoEMethod and GPTQMarlinMoEMethod create_weights / process_weights_after_loading
    / apply (awq_marlin.py:506-735, gptq_marlin.py:590-931).

Checkpoint tensors are plain torch parameters in their checkpoint layouts (the reference's
BasevLLMParameter / weight-loader machinery belongs to the serving engine, outside this
path):
  GPTQ  qweight [K/pack, N] int32 packed along K; scales [G, N]; qzeros [G, N/pack] packed
        along N; g_idx [K] (act-order).
  AWQ   qweight [K, N/pack] int32 packed along N in AWQ order [0,2,4,6,1,3,5,7] ([0,2,1,3] for
        8 bits); qzeros [G, N/pack] in the same order; scales [G, N].
  MoE   the same per expert, with the reference's shapes: AWQ w13_qweight [E, H, 2I/pack],
        w2_qweight [E, I, H/pack]; GPTQ w13_qweight [E, H/pack, 2I], w2_qweight [E, I/pack, H].

As in the reference, integer zero points of uint4 / uint8 weights are turned into float zero
points dtype(z * s) at load time (marlin.py:166-191; awq_marlin.py:701-725), and act-order is
applied by repacking with argsort(g_idx) (marlin.py:151-159).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _custom_ops as ops
from .fused_marlin_moe import fused_marlin_moe
from .marlin_utils import (MARLIN_SUPPORTED_GROUP_SIZES, apply_gptq_marlin_linear,
                           marlin_is_k_full, marlin_logical_scales, marlin_make_empty_g_idx,
                           marlin_make_workspace_new, marlin_moe_logical_scales,
                           marlin_permute_bias, marlin_sort_g_idx,
                           moe_awq_to_marlin_zero_points_float, unpack_cols)
from .scalar_type import ScalarType, scalar_types

AWQ_PACK_ORDER = {4: [0, 2, 4, 6, 1, 3, 5, 7], 8: [0, 2, 1, 3]}


def _replace(layer: torch.nn.Module, name: str, value: torch.Tensor) -> None:
    """replace_parameter (vllm/model_executor/layers/quantization/utils/__init__.py)."""
    if name in layer._parameters:
        del layer._parameters[name]
    layer.register_parameter(name, torch.nn.Parameter(value, requires_grad=False))


def query_marlin_supported_quant_types(has_zp: bool) -> list[ScalarType]:
    """marlin_utils.py query_marlin_supported_quant_types (16-bit activations)."""
    if has_zp:
        return [scalar_types.uint4, scalar_types.uint8]
    return [scalar_types.uint4b8, scalar_types.uint8b128]


def check_marlin_supports_shape(output_size_per_partition: int, input_size_per_partition: int,
                                input_size: int, group_size: int) -> tuple[bool, str | None]:
    """The shape rules of the ops: N % 64, K % 32 (the gfx950 layout), K % group_size."""
    if output_size_per_partition % 64 != 0:
        return False, (f"output_size_per_partition = {output_size_per_partition} is not "
                       "divisible by min_thread_n = 64")
    if input_size_per_partition % 32 != 0:
        return False, (f"input_size_per_partition = {input_size_per_partition} is not "
                       "divisible by 32")
    if group_size < input_size and group_size != -1 and input_size_per_partition % group_size:
        return False, (f"input_size_per_partition = {input_size_per_partition} is not "
                       f"divisible by group_size = {group_size}")
    return True, None


@dataclass
class MPLinearLayerConfig:
    """MPLinearKernel.py:14-24."""
    full_weight_shape: tuple[int, int]  # [in, out]
    partition_weight_shape: tuple[int, int]
    weight_type: ScalarType
    act_type: torch.dtype
    group_size: int
    zero_points: bool
    has_g_idx: bool
    out_type: torch.dtype | None = None


class MarlinLinearKernel:
    """The reference's MarlinLinearKernel (marlin.py:30-214) on this build.  Parameters named
    by the caller hold the GPTQ-layout checkpoint tensors; process_weights_after_loading
    rewrites them into the op formats, apply_weights runs marlin_gemm."""

    @classmethod
    def get_min_capability(cls) -> int:
        return 70

    @classmethod
    def can_implement(cls, c: MPLinearLayerConfig) -> tuple[bool, str | None]:
        if c.act_type not in (torch.float16, torch.bfloat16):
            return False, "only float16 and bfloat16 activations are supported on this build"
        quant_types = query_marlin_supported_quant_types(c.zero_points)
        if c.weight_type not in quant_types:
            return False, (f"Quant type ({c.weight_type}) not supported by Marlin, supported "
                           f"types are: {quant_types}")
        if c.group_size not in MARLIN_SUPPORTED_GROUP_SIZES:
            return False, (f"Group size ({c.group_size}) not supported by Marlin, supported "
                           f"group sizes are: {MARLIN_SUPPORTED_GROUP_SIZES}")
        return check_marlin_supports_shape(c.partition_weight_shape[1],
                                           c.partition_weight_shape[0], c.full_weight_shape[0],
                                           c.group_size)

    def __init__(self, c: MPLinearLayerConfig, w_q_param_name: str, w_s_param_name: str,
                 w_zp_param_name: str | None = None, w_gidx_param_name: str | None = None):
        ok, why = self.can_implement(c)
        if not ok:
            raise ValueError(why)
        self.config = c
        self.w_q_name = w_q_param_name
        self.w_s_name = w_s_param_name
        if c.zero_points:
            assert w_zp_param_name is not None
        if c.has_g_idx:
            assert w_gidx_param_name is not None
        self.w_zp_name = w_zp_param_name
        self.w_gidx_name = w_gidx_param_name
        self.is_k_full = True
        self.is_zp_float = False
        self.workspace: torch.Tensor | None = None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        c = self.config
        device = getattr(layer, self.w_q_name).device
        size_k, size_n = c.partition_weight_shape
        row_parallel = c.partition_weight_shape[0] != c.full_weight_shape[0]
        self.is_k_full = marlin_is_k_full(c.has_g_idx, row_parallel)
        self.workspace = marlin_make_workspace_new(device)
        if self.w_gidx_name is None:
            self.w_gidx_name = "g_idx"
        if self.w_zp_name is None:
            self.w_zp_name = "w_zp"

        if c.has_g_idx:
            g_idx, sort_indices = marlin_sort_g_idx(getattr(layer, self.w_gidx_name).data)
            _replace(layer, self.w_gidx_name, g_idx)
            layer.g_idx_sort_indices = sort_indices
        else:
            setattr(layer, self.w_gidx_name, marlin_make_empty_g_idx(device))
            layer.g_idx_sort_indices = marlin_make_empty_g_idx(device)

        grouped_k = size_k // c.group_size if c.group_size != -1 else 1
        scales = getattr(layer, self.w_s_name).data.contiguous().reshape(grouped_k, size_n)
        if c.zero_points:
            # integer zero points -> float zero points dtype(z * s) (marlin.py:166-191)
            zp = unpack_cols(getattr(layer, self.w_zp_name).data, c.weight_type.size_bits,
                             grouped_k, size_n)
            zp_float = (zp.to(torch.float32) * scales.to(torch.float32)).to(scales.dtype)
            _replace(layer, self.w_zp_name,
                     marlin_logical_scales(zp_float, size_k, size_n, c.group_size))
            self.is_zp_float = True
        else:
            setattr(layer, self.w_zp_name, marlin_make_empty_g_idx(device))

        _replace(layer, self.w_q_name,
                 ops.gptq_marlin_repack(getattr(layer, self.w_q_name).data.contiguous(),
                                        layer.g_idx_sort_indices, size_k, size_n,
                                        c.weight_type.size_bits))
        _replace(layer, self.w_s_name, marlin_logical_scales(scales, size_k, size_n, c.group_size))
        if getattr(layer, "bias", None) is not None:
            layer.bias.data = marlin_permute_bias(layer.bias.data)

    def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor,
                      bias: torch.Tensor | None = None) -> torch.Tensor:
        c = self.config
        if (self.workspace is None or self.workspace.device != x.device
                or self.workspace.numel() != 0):
            self.workspace = marlin_make_workspace_new(x.device)
        w_zp = getattr(layer, self.w_zp_name, None)
        return apply_gptq_marlin_linear(
            input=x, weight=getattr(layer, self.w_q_name), weight_scale=getattr(layer, self.w_s_name),
            weight_zp=w_zp, g_idx=getattr(layer, self.w_gidx_name, None),
            g_idx_sort_indices=layer.g_idx_sort_indices, workspace=self.workspace,
            wtype=c.weight_type, output_size_per_partition=c.partition_weight_shape[1],
            input_size_per_partition=c.partition_weight_shape[0], is_k_full=self.is_k_full,
            bias=bias, is_zp_float=self.is_zp_float)


def convert_awq_to_standard_format(layer: torch.nn.Module, w_q_name: str, w_zp_name: str,
                                   size_bits: int) -> None:
    """AWQ qweight [K, N/pack] (AWQ order, packed along N) -> GPTQ-like [K/pack, N] packed
    along K in natural order; qzeros [G, N/pack] -> natural order along N
    (awq_marlin.py:75-130)."""
    pack = 32 // size_bits
    mask = (1 << size_bits) - 1
    qw = getattr(layer, w_q_name).data
    device = qw.device
    undo = torch.argsort(torch.tensor(AWQ_PACK_ORDER[size_bits])).to(device)
    shifts = torch.arange(0, 32, size_bits, dtype=torch.int64, device=device)

    def unpack_awq(words: torch.Tensor) -> torch.Tensor:  # [R, C/pack] -> [R, C] natural
        vals = (words.to(torch.int64).unsqueeze(-1) >> shifts) & mask
        return vals[:, :, undo].reshape(words.shape[0], -1)

    k = qw.shape[0]
    vals = unpack_awq(qw)  # [K, N]
    n = vals.shape[1]
    packed = (vals.reshape(k // pack, pack, n) << shifts[None, :, None]).sum(dim=1)
    packed = torch.where(packed >= 2 ** 31, packed - 2 ** 32, packed).to(torch.int32)
    _replace(layer, w_q_name, packed.contiguous())

    zp = getattr(layer, w_zp_name, None)
    if zp is not None:
        zvals = unpack_awq(zp.data)
        g = zvals.shape[0]
        zpk = (zvals.reshape(g, n // pack, pack) << shifts[None, None, :]).sum(dim=2)
        zpk = torch.where(zpk >= 2 ** 31, zpk - 2 ** 32, zpk).to(torch.int32)
        _replace(layer, w_zp_name, zpk.contiguous())


@dataclass
class AWQMarlinConfig:
    """The parts of the reference's AWQMarlinConfig the methods read."""
    weight_bits: int = 4
    group_size: int = 128
    zero_point: bool = True

    @property
    def pack_factor(self) -> int:
        return 32 // self.weight_bits

    @property
    def quant_type(self) -> ScalarType:
        return {4: scalar_types.uint4, 8: scalar_types.uint8}[self.weight_bits]


@dataclass
class GPTQMarlinConfig:
    """The parts of the reference's GPTQMarlinConfig the methods read (symmetric GPTQ)."""
    weight_bits: int = 4
    group_size: int = 128
    desc_act: bool = False

    @property
    def pack_factor(self) -> int:
        return 32 // self.weight_bits

    @property
    def quant_type(self) -> ScalarType:
        return {4: scalar_types.uint4b8, 8: scalar_types.uint8b128}[self.weight_bits]


class AWQMarlinLinearMethod:
    """awq_marlin.py:355-483: AWQ checkpoint tensors, converted to the GPTQ-like layout and
    handed to MarlinLinearKernel."""

    def __init__(self, quant_config: AWQMarlinConfig):
        self.quant_config = quant_config

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: list[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, device: torch.device | str = "cuda") -> None:
        qc = self.quant_config
        n = sum(output_partition_sizes)
        gs = qc.group_size if qc.group_size != -1 else input_size
        cfg = MPLinearLayerConfig((input_size, output_size), (input_size_per_partition, n),
                                  qc.quant_type, params_dtype, qc.group_size, qc.zero_point, False)
        groups = input_size_per_partition // gs
        layer.register_parameter("qweight", torch.nn.Parameter(torch.empty(
            (input_size_per_partition, n // qc.pack_factor), dtype=torch.int32, device=device),
            requires_grad=False))
        layer.register_parameter("qzeros", torch.nn.Parameter(torch.empty(
            (groups, n // qc.pack_factor), dtype=torch.int32, device=device), requires_grad=False))
        layer.register_parameter("scales", torch.nn.Parameter(torch.empty(
            (groups, n), dtype=params_dtype, device=device), requires_grad=False))
        self.kernel = MarlinLinearKernel(cfg, "qweight", "scales", "qzeros")

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        convert_awq_to_standard_format(layer, "qweight", "qzeros",
                                       self.quant_config.quant_type.size_bits)
        self.kernel.process_weights_after_loading(layer)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: torch.Tensor | None = None) -> torch.Tensor:
        return self.kernel.apply_weights(layer, x, bias)


class AWQMarlinMoEMethod:
    """awq_marlin.py:485-735 (16-bit activations)."""

    def __init__(self, quant_config: AWQMarlinConfig):
        if quant_config.weight_bits not in (4, 8):
            raise ValueError("AWQMarlinMoEMethod only supports 4-bit and 8-bit weights now.")
        self.quant_config = quant_config
        self.quant_type = quant_config.quant_type

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype,
                       device: torch.device | str = "cuda") -> None:
        qc = self.quant_config
        inter = intermediate_size_per_partition
        layer.intermediate_size_per_partition = inter
        g13 = 1 if qc.group_size == -1 else hidden_size // qc.group_size
        g2 = 1 if qc.group_size == -1 else inter // qc.group_size
        layer.num_groups_w13, layer.num_groups_w2 = g13, g2
        p = qc.pack_factor

        def reg(name, shape, dtype):
            layer.register_parameter(name, torch.nn.Parameter(
                torch.empty(shape, dtype=dtype, device=device), requires_grad=False))

        reg("w13_qweight", (num_experts, hidden_size, 2 * inter // p), torch.int32)
        reg("w2_qweight", (num_experts, inter, hidden_size // p), torch.int32)
        reg("w13_scales", (num_experts, g13, 2 * inter), params_dtype)
        reg("w2_scales", (num_experts, g2, hidden_size), params_dtype)
        reg("w13_qzeros", (num_experts, g13, 2 * inter // p), torch.int32)
        reg("w2_qzeros", (num_experts, g2, hidden_size // p), torch.int32)
        layer.workspace = marlin_make_workspace_new(torch.device(device), 4)

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        qc = self.quant_config
        num_experts = layer.w13_qweight.shape[0]
        device = layer.w13_qweight.device
        empty = torch.empty((num_experts, 0), dtype=torch.int32, device=device)
        layer.w13_g_idx_sort_indices = torch.nn.Parameter(empty, requires_grad=False)
        layer.w2_g_idx_sort_indices = torch.nn.Parameter(empty.clone(), requires_grad=False)
        _replace(layer, "w13_qweight", ops.awq_marlin_moe_repack(
            layer.w13_qweight, layer.w13_g_idx_sort_indices,
            size_k=layer.w13_qweight.shape[1], size_n=layer.w13_qweight.shape[2] * qc.pack_factor,
            num_bits=qc.weight_bits))
        _replace(layer, "w2_qweight", ops.awq_marlin_moe_repack(
            layer.w2_qweight, layer.w2_g_idx_sort_indices,
            size_k=layer.w2_qweight.shape[1], size_n=layer.w2_qweight.shape[2] * qc.pack_factor,
            num_bits=qc.weight_bits))
        layer.w13_weight, layer.w2_weight = layer.w13_qweight, layer.w2_qweight
        w13_scales = layer.w13_scales.data.contiguous()
        w2_scales = layer.w2_scales.data.contiguous()
        inter = layer.intermediate_size_per_partition
        _replace(layer, "w13_scales", marlin_moe_logical_scales(
            w13_scales, inter, w13_scales.shape[2], qc.group_size))
        _replace(layer, "w2_scales", marlin_moe_logical_scales(
            w2_scales, inter, w2_scales.shape[2], qc.group_size))
        _replace(layer, "w13_qzeros", moe_awq_to_marlin_zero_points_float(
            layer.w13_qzeros, w13_scales, size_k=layer.w13_qzeros.shape[1],
            size_n=layer.w13_qzeros.shape[2] * qc.pack_factor, num_bits=qc.weight_bits,
            scale_size_k=inter, group_size=qc.group_size))
        _replace(layer, "w2_qzeros", moe_awq_to_marlin_zero_points_float(
            layer.w2_qzeros, w2_scales, size_k=layer.w2_qzeros.shape[1],
            size_n=layer.w2_qzeros.shape[2] * qc.pack_factor, num_bits=qc.weight_bits,
            scale_size_k=inter, group_size=qc.group_size))
        for name in ("w13_bias", "w2_bias"):
            if getattr(layer, name, None) is not None:
                getattr(layer, name).data = marlin_permute_bias(getattr(layer, name).data)
        layer.workspace = marlin_make_workspace_new(device, 4)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, topk_weights: torch.Tensor,
              topk_ids: torch.Tensor, expert_map: torch.Tensor | None = None,
              global_num_experts: int = -1,
              apply_router_weight_on_input: bool = False) -> torch.Tensor:
        return fused_marlin_moe(
            x, layer.w13_qweight, layer.w2_qweight, getattr(layer, "w13_bias", None),
            getattr(layer, "w2_bias", None), layer.w13_scales, layer.w2_scales, topk_weights,
            topk_ids, quant_type_id=self.quant_type.id,
            apply_router_weight_on_input=apply_router_weight_on_input,
            global_num_experts=global_num_experts, expert_map=expert_map,
            w1_zeros=layer.w13_qzeros, w2_zeros=layer.w2_qzeros, is_w1_zp_float=True,
            is_w2_zp_float=True, workspace=layer.workspace)


class GPTQMarlinMoEMethod:
    """gptq_marlin.py:590-931 (symmetric GPTQ, 16-bit activations).  Act-order MoE weights
    are rejected by the MoE GEMM op, as in the reference (ops.cu:126-128)."""

    def __init__(self, quant_config: GPTQMarlinConfig):
        self.quant_config = quant_config
        self.quant_type = quant_config.quant_type
        self.is_k_full = True

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype,
                       intermediate_size_full: int | None = None,
                       device: torch.device | str = "cuda") -> None:
        qc = self.quant_config
        inter = intermediate_size_per_partition
        self.is_k_full = (intermediate_size_full or inter) == inter
        layer.intermediate_size_per_partition = inter
        g13 = 1 if qc.group_size == -1 else hidden_size // qc.group_size
        g2 = 1 if qc.group_size == -1 else inter // qc.group_size
        layer.num_groups_w13, layer.num_groups_w2 = g13, g2
        p = qc.pack_factor

        def reg(name, shape, dtype):
            layer.register_parameter(name, torch.nn.Parameter(
                torch.empty(shape, dtype=dtype, device=device), requires_grad=False))

        reg("w13_qweight", (num_experts, hidden_size // p, 2 * inter), torch.int32)
        reg("w2_qweight", (num_experts, inter // p, hidden_size), torch.int32)
        reg("w13_scales", (num_experts, g13, 2 * inter), params_dtype)
        reg("w2_scales", (num_experts, g2, hidden_size), params_dtype)
        reg("w13_g_idx", (num_experts, hidden_size), torch.int32)
        reg("w2_g_idx", (num_experts, inter), torch.int32)
        layer.workspace = marlin_make_workspace_new(torch.device(device), 4)

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        qc = self.quant_config
        num_experts = layer.w13_g_idx.shape[0]
        device = layer.w13_g_idx.device
        if qc.desc_act:
            sorted13, idx13, sorted2, idx2 = [], [], [], []
            for e in range(num_experts):
                g, i = marlin_sort_g_idx(layer.w13_g_idx[e])
                sorted13.append(g)
                idx13.append(i)
                g, i = marlin_sort_g_idx(layer.w2_g_idx[e])
                sorted2.append(g)
                idx2.append(i)
            _replace(layer, "w13_g_idx", torch.stack(sorted13))
            _replace(layer, "w2_g_idx", torch.stack(sorted2))
            layer.w13_g_idx_sort_indices = torch.nn.Parameter(torch.stack(idx13),
                                                              requires_grad=False)
            layer.w2_g_idx_sort_indices = torch.nn.Parameter(torch.stack(idx2),
                                                             requires_grad=False)
        else:
            empty = torch.empty((num_experts, 0), dtype=torch.int32, device=device)
            _replace(layer, "w13_g_idx", empty)
            _replace(layer, "w2_g_idx", empty.clone())
            layer.w13_g_idx_sort_indices = torch.nn.Parameter(empty.clone(), requires_grad=False)
            layer.w2_g_idx_sort_indices = torch.nn.Parameter(empty.clone(), requires_grad=False)
        _replace(layer, "w13_qweight", ops.gptq_marlin_moe_repack(
            layer.w13_qweight, layer.w13_g_idx_sort_indices,
            layer.w13_qweight.shape[1] * qc.pack_factor, layer.w13_qweight.shape[2],
            qc.weight_bits))
        _replace(layer, "w2_qweight", ops.gptq_marlin_moe_repack(
            layer.w2_qweight, layer.w2_g_idx_sort_indices,
            layer.w2_qweight.shape[1] * qc.pack_factor, layer.w2_qweight.shape[2],
            qc.weight_bits))
        layer.w13_weight, layer.w2_weight = layer.w13_qweight, layer.w2_qweight
        inter = layer.intermediate_size_per_partition
        _replace(layer, "w13_scales", marlin_moe_logical_scales(
            layer.w13_scales.data, inter, layer.w13_scales.shape[2], qc.group_size))
        _replace(layer, "w2_scales", marlin_moe_logical_scales(
            layer.w2_scales.data, inter, layer.w2_scales.shape[2], qc.group_size))
        for name in ("w13_bias", "w2_bias"):
            if getattr(layer, name, None) is not None:
                getattr(layer, name).data = marlin_permute_bias(getattr(layer, name).data)
        layer.workspace = marlin_make_workspace_new(device, 4)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, topk_weights: torch.Tensor,
              topk_ids: torch.Tensor, expert_map: torch.Tensor | None = None,
              global_num_experts: int = -1,
              apply_router_weight_on_input: bool = False) -> torch.Tensor:
        return fused_marlin_moe(
            x, layer.w13_qweight, layer.w2_qweight, getattr(layer, "w13_bias", None),
            getattr(layer, "w2_bias", None), layer.w13_scales, layer.w2_scales, topk_weights,
            topk_ids, quant_type_id=self.quant_type.id,
            apply_router_weight_on_input=apply_router_weight_on_input,
            global_num_experts=global_num_experts, expert_map=expert_map,
            g_idx1=layer.w13_g_idx, g_idx2=layer.w2_g_idx,
            sort_indices1=layer.w13_g_idx_sort_indices,
            sort_indices2=layer.w2_g_idx_sort_indices, workspace=layer.workspace,
            is_k_full=self.is_k_full)
