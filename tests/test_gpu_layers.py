"""GPU parity of the layer-integration steps (marlin_v100_amd/layers.py): checkpoint-format
GPTQ / AWQ tensors go through process_weights_after_loading and apply exactly as the
reference's MarlinLinearKernel / AWQMarlinLinearMethod / AWQ- and GPTQMarlinMoEMethod do
(marlin.py:68-214, awq_marlin.py:75-130, 355-735, gptq_marlin.py:590-931), and the result
matches the oracle's dequantize-then-matmul of the same checkpoint within the north-star
tolerance.  The oracle builds the checkpoints from logical codes, so every packing order and
metadata conversion on the way is checked end to end."""
import pytest
import torch

import oracle as O
from marlin_v100_amd.layers import (AWQMarlinConfig, AWQMarlinLinearMethod, AWQMarlinMoEMethod,
                                    GPTQMarlinConfig, GPTQMarlinMoEMethod, MarlinLinearKernel,
                                    MPLinearLayerConfig)
from marlin_v100_amd.scalar_type import scalar_types

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _param(t):
    return torch.nn.Parameter(t.cuda(), requires_grad=False)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_marlin_linear_kernel_gptq_act_order_with_bias(dtype):
    k, n, gs, m = 1024, 256, 128, 16
    gen = torch.Generator().manual_seed(21)
    g_idx = O.act_order_groups(k, gs, gen)
    w = (torch.randn((k, n), generator=gen) * 0.02).to(dtype)
    q, s, _z, _zp = O.quantize_g_idx(w, g_idx, k // gs, "u4b8", dtype)
    bias = (torch.randn(n, generator=gen) * 0.1).to(dtype)
    layer = torch.nn.Module()
    layer.qweight = _param(O.gptq_pack(q, 4))
    layer.scales = _param(s)
    layer.g_idx = _param(g_idx)
    layer.bias = _param(bias)
    cfg = MPLinearLayerConfig((k, n), (k, n), scalar_types.uint4b8, dtype, gs, False, True)
    kernel = MarlinLinearKernel(cfg, "qweight", "scales", None, "g_idx")
    kernel.process_weights_after_loading(layer)
    x = torch.randn((2, m // 2, k), generator=gen).to(dtype)
    out = kernel.apply_weights(layer, x.cuda(), layer.bias).cpu()
    assert out.shape == (2, m // 2, n)
    deq = O.dequant_int_g_idx(q, s, "u4b8", dtype, g_idx)
    ref = O.gemm_ref(x.reshape(m, k), deq, bias).reshape(2, m // 2, n)
    assert O.max_abs_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [4, 8])
def test_marlin_linear_kernel_zero_points(dtype, bits):
    """GPTQ-layout uint4 / uint8 with integer zero points: converted to float zero points
    dtype(z * s) at load time, as the reference does (marlin.py:166-191)."""
    k, n, gs, m = 512, 256, 128, 5
    gen = torch.Generator().manual_seed(22 + bits)
    w = (torch.randn((k, n), generator=gen) * 0.02).to(dtype)
    q, s, z, zp_f = O.quantize_with_zero_point(w, gs, bits, dtype)
    layer = torch.nn.Module()
    layer.qweight = _param(O.gptq_pack(q, bits))
    layer.scales = _param(s)
    layer.qzeros = _param(O.pack_cols(z, bits))
    wtype = scalar_types.uint4 if bits == 4 else scalar_types.uint8
    cfg = MPLinearLayerConfig((k, n), (k, n), wtype, dtype, gs, True, False)
    kernel = MarlinLinearKernel(cfg, "qweight", "scales", "qzeros")
    kernel.process_weights_after_loading(layer)
    x = torch.randn((m, k), generator=gen).to(dtype)
    out = kernel.apply_weights(layer, x.cuda()).cpu()
    ref = O.gemm_ref(x, O.dequant_int(q, s, "u4" if bits == 4 else "u8", dtype, zp_f))
    assert O.max_abs_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_awq_marlin_linear_method(dtype):
    k, n, gs, m = 512, 320, 128, 33
    gen = torch.Generator().manual_seed(23)
    w = (torch.randn((k, n), generator=gen) * 0.02).to(dtype)
    q, s, z, zp_f = O.quantize_with_zero_point(w, gs, 4, dtype)
    method = AWQMarlinLinearMethod(AWQMarlinConfig(4, gs, True))
    layer = torch.nn.Module()
    method.create_weights(layer, k, [n], k, n, dtype)
    layer.qweight.data.copy_(O.awq_pack(q, 4))
    layer.qzeros.data.copy_(O.awq_pack(z, 4))
    layer.scales.data.copy_(s)
    method.process_weights_after_loading(layer)
    x = torch.randn((m, k), generator=gen).to(dtype)
    out = method.apply(layer, x.cuda()).cpu()
    ref = O.gemm_ref(x, O.dequant_int(q, s, "u4", dtype, zp_f))
    assert O.max_abs_rel_err(out, ref) <= TOL


def _experts(fmt, e, k, n, dtype, seed, gs=128):
    gen = torch.Generator().manual_seed(seed)
    qs, ss, zs, deqs = [], [], [], []
    for _ in range(e):
        w = (torch.randn((k, n), generator=gen) * 0.02).to(dtype)
        if fmt == "u4":
            q, s, z, zp_f = O.quantize_with_zero_point(w, gs, 4, dtype)
            deqs.append(O.dequant_int(q, s, "u4", dtype, zp_f))
        else:
            q, s = O.quantize_with_bias(w, gs, 8, dtype)
            z = None
            deqs.append(O.dequant_int(q, s, "u4b8", dtype))
        qs.append(q)
        ss.append(s)
        zs.append(z)
    return qs, ss, zs, torch.stack(deqs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tokens", [8, 96])
def test_awq_marlin_moe_method(dtype, tokens):
    E, topk, H, I = 8, 2, 256, 128
    q13, s13, z13, d13 = _experts("u4", E, H, 2 * I, dtype, 31)
    q2, s2, z2, d2 = _experts("u4", E, I, H, dtype, 32)
    method = AWQMarlinMoEMethod(AWQMarlinConfig(4, 128, True))
    layer = torch.nn.Module()
    method.create_weights(layer, E, H, I, dtype)
    for e in range(E):
        layer.w13_qweight.data[e].copy_(O.awq_pack(q13[e], 4))
        layer.w13_qzeros.data[e].copy_(O.awq_pack(z13[e], 4))
        layer.w13_scales.data[e].copy_(s13[e])
        layer.w2_qweight.data[e].copy_(O.awq_pack(q2[e], 4))
        layer.w2_qzeros.data[e].copy_(O.awq_pack(z2[e], 4))
        layer.w2_scales.data[e].copy_(s2[e])
    method.process_weights_after_loading(layer)
    gen = torch.Generator().manual_seed(33)
    x = torch.randn((tokens, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((tokens, E), generator=gen), topk)
    out = method.apply(layer, x.cuda(), tw.cuda(), ids.cuda()).cpu()
    ref = O.moe_layer_ref(x, d13, d2, tw, ids)
    assert O.max_abs_rel_err(out, ref) <= 2 * TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gptq_marlin_moe_method(dtype):
    E, topk, H, I, tokens = 8, 2, 256, 128, 40
    q13, s13, _z, d13 = _experts("u4b8", E, H, 2 * I, dtype, 41)
    q2, s2, _z2, d2 = _experts("u4b8", E, I, H, dtype, 42)
    method = GPTQMarlinMoEMethod(GPTQMarlinConfig(4, 128, False))
    layer = torch.nn.Module()
    method.create_weights(layer, E, H, I, dtype)
    for e in range(E):
        layer.w13_qweight.data[e].copy_(O.gptq_pack(q13[e], 4))
        layer.w13_scales.data[e].copy_(s13[e])
        layer.w2_qweight.data[e].copy_(O.gptq_pack(q2[e], 4))
        layer.w2_scales.data[e].copy_(s2[e])
    method.process_weights_after_loading(layer)
    gen = torch.Generator().manual_seed(43)
    x = torch.randn((tokens, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((tokens, E), generator=gen), topk)
    out = method.apply(layer, x.cuda(), tw.cuda(), ids.cuda()).cpu()
    ref = O.moe_layer_ref(x, d13, d2, tw, ids)
    assert O.max_abs_rel_err(out, ref) <= 2 * TOL
