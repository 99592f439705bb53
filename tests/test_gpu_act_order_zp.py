"""GPU parity of the two marlin_gemm modes the SM70 reference rejects and upstream marlin
takes (reference marlin.cu:95-102, 336-339; upstream marlin_utils.py:274-276, 347-396):

* packed integer zero points (is_zp_float=False): the weights dequantize to the single
  rounding of (q - z) * s, bit-exact through the dequantize op, and the GEMM is within the
  north-star tolerance of A @ that;
* act-order: weights repacked with perm = argsort(g_idx), A gathered by perm, the sorted
  g_idx passed with it; the result is within tolerance of A @ W with every row's scale taken
  from its own group (the oracle never permutes anything), and a g_idx whose groups do not
  hold group_size rows comes out NaN instead of silently wrong."""
import pytest
import torch

import oracle as O
from marlin_v100_amd import _custom_ops as ops
from marlin_v100_amd import capi
from marlin_v100_amd.marlin_utils import marlin_sort_g_idx, marlin_zero_points
from marlin_v100_amd.scalar_type import scalar_types
from tests.quant_cases import TYPE_ID

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _int_zp_case(fmt, k, n, gs, dtype, seed):
    bits = 4 if fmt == "u4" else 8
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn((k, n), generator=gen) * 0.02).to(dtype)
    q, s, z, _zp = O.quantize_with_zero_point(w, gs, bits, dtype)
    return q, s, z, bits


@pytest.mark.parametrize("fmt", ["u4", "u8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("gs", [-1, 64, 128])
def test_int_zero_point_dequant_bit_exact(fmt, dtype, gs):
    k, n = 512, 256
    print(f"case int-zp dequant fmt={fmt} dtype={dtype} gs={gs}", flush=True)
    q, s, z, bits = _int_zp_case(fmt, k, n, gs, dtype, seed=gs + 7)
    words = capi.gptq_marlin_repack(O.gptq_pack(q, bits).cuda(), None, k, n, bits)
    zp = O.pack_cols(z, bits).cuda()
    out = capi.dequantize(words, s.cuda(), TYPE_ID[fmt], k, n, dtype, b_zeros=zp).cpu()
    ref = O.dequant_int_zero(q, s, z, dtype)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("fmt", ["u4", "u8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 16, 64, 200])
@pytest.mark.parametrize("gs", [-1, 32, 128])
def test_gemm_int_zero_points(fmt, dtype, m, gs):
    k, n = 1024, 256 if m != 200 else 320
    print(f"case int-zp gemm fmt={fmt} dtype={dtype} m={m} gs={gs}", flush=True)
    q, s, z, bits = _int_zp_case(fmt, k, n, gs, dtype, seed=m * 31 + gs)
    words = capi.gptq_marlin_repack(O.gptq_pack(q, bits).cuda(), None, k, n, bits)
    zp = O.pack_cols(z, bits).cuda()
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(m)).to(dtype)
    out = capi.marlin_gemm(a.cuda(), words, s.cuda(), TYPE_ID[fmt], m, n, k, b_zeros=zp,
                           is_zp_float=False).cpu()
    ref = O.gemm_ref(a, O.dequant_int_zero(q, s, z, dtype))
    assert O.max_abs_rel_err(out, ref) <= TOL


def test_int_zero_points_through_torch_op_and_utils():
    """ops.marlin_gemm with the int32 zero points marlin_zero_points() produces."""
    k, n, m = 1024, 512, 8
    q, s, z, bits = _int_zp_case("u4", k, n, 128, torch.float16, seed=3)
    words = ops.gptq_marlin_repack(O.gptq_pack(q, 4).cuda(),
                                   torch.empty(0, dtype=torch.int32, device="cuda"), k, n, 4)
    zp = marlin_zero_points(z.cuda(), k // 128, n, 4)
    assert torch.equal(zp.cpu(), O.pack_cols(z, 4))
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(9)).half()
    ws = torch.empty(0, dtype=torch.int32, device="cuda")
    out = ops.marlin_gemm(a.cuda(), None, words, None, s.cuda(), None, None, zp, None, None, ws,
                          scalar_types.uint4, m, n, k, is_zp_float=False).cpu()
    assert O.max_abs_rel_err(out, O.gemm_ref(a, O.dequant_int_zero(q, s, z, torch.float16))) <= TOL


def _act_order_case(fmt, k, n, gs, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    ngroups = 1 if gs == -1 else k // gs
    g_idx = O.act_order_groups(k, k if gs == -1 else gs, gen)
    w = (torch.randn((k, n), generator=gen) * 0.02).to(dtype)
    q, s, z, zp_f = O.quantize_g_idx(w, g_idx, ngroups, fmt, dtype)
    deq = O.dequant_int_g_idx(q, s, fmt, dtype, g_idx, zp_f)
    return g_idx, q, s, zp_f, deq


@pytest.mark.parametrize("fmt", ["u4b8", "u4", "u8b128"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 16, 200])
@pytest.mark.parametrize("gs", [-1, 64, 128])
def test_gemm_act_order(fmt, dtype, m, gs):
    k, n = 1024, 256
    bits = 4 if fmt in ("u4b8", "u4") else 8
    print(f"case act-order fmt={fmt} dtype={dtype} m={m} gs={gs}", flush=True)
    g_idx, q, s, zp_f, deq = _act_order_case(fmt, k, n, gs, dtype, seed=m + gs + 11)
    g_sorted, perm = marlin_sort_g_idx(g_idx)
    words = capi.gptq_marlin_repack(O.gptq_pack(q, bits).cuda(), perm.cuda(), k, n, bits)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(m + 1)).to(dtype)
    out = capi.marlin_gemm(a.cuda(), words, s.cuda(), TYPE_ID[fmt], m, n, k,
                           b_zeros=None if zp_f is None else zp_f.cuda(),
                           is_zp_float=zp_f is not None, g_idx=g_sorted.cuda(),
                           perm=perm.cuda()).cpu()
    assert O.max_abs_rel_err(out, O.gemm_ref(a, deq)) <= TOL


def test_act_order_strided_a_and_torch_op():
    """A with a row stride > K, through the torch op, twice in a row (staging buffer reuse)."""
    k, n, m = 512, 256, 24
    g_idx, q, s, _zpf, deq = _act_order_case("u4b8", k, n, 128, torch.bfloat16, seed=5)
    g_sorted, perm = marlin_sort_g_idx(g_idx)
    ws = torch.empty(0, dtype=torch.int32, device="cuda")
    words = ops.gptq_marlin_repack(O.gptq_pack(q, 4).cuda(), perm.cuda(), k, n, 4)
    big = torch.randn((m, k + 64), generator=torch.Generator().manual_seed(2)).bfloat16()
    a = big[:, :k]
    for _ in range(2):
        out = ops.marlin_gemm(big.cuda()[:, :k], None, words, None, s.cuda(), None, None, None,
                              g_sorted.cuda(), perm.cuda(), ws, scalar_types.uint4b8, m, n, k,
                              is_k_full=True).cpu()
        assert O.max_abs_rel_err(out, O.gemm_ref(a, deq)) <= TOL


def test_act_order_bad_groups_come_out_nan():
    k, n, m = 512, 256, 4
    g_idx, q, s, _zpf, _deq = _act_order_case("u4b8", k, n, 128, torch.float16, seed=8)
    g_sorted, perm = marlin_sort_g_idx(g_idx)
    bad = g_sorted.clone()
    bad[5] = 1  # row 5 sits in group 0 of the sorted order
    words = capi.gptq_marlin_repack(O.gptq_pack(q, 4).cuda(), perm.cuda(), k, n, 4)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(4)).half()
    out = capi.marlin_gemm(a.cuda(), words, s.cuda(), TYPE_ID["u4b8"], m, n, k,
                           g_idx=bad.cuda(), perm=perm.cuda()).cpu()
    assert torch.isnan(out).all()
    bad_perm = perm.clone()
    bad_perm[7] = k + 3  # out of range: never read, comes out NaN
    out = capi.marlin_gemm(a.cuda(), words, s.cuda(), TYPE_ID["u4b8"], m, n, k,
                           g_idx=g_sorted.cuda(), perm=bad_perm.cuda()).cpu()
    assert torch.isnan(out).all()
