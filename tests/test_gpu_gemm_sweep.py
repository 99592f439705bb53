"""Seeded random sweep of marlin_gemm against the oracle (dequantize, fp32 matmul): every
format, both dtypes, the group sizes each format allows, M from 1 to ~700 (log-uniform), N any
multiple of 64 up to 2048 and K any multiple of the group size (so K tails, column counts that
are not multiples of 128 or 256, and every selector regime: decode, multistage, 128-row and
tiled kernels, split K), a permuted bias on about a third of the cases.  The bar is the
north-star tolerance max|out - ref| <= 1e-2 * max|ref|; the case parameters are printed
before each launch."""
import math
import random

import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from marlin_v100_amd.marlin_utils import marlin_sort_g_idx
from tests.quant_cases import BITS, FORMATS, TYPE_ID, make_case, to_dev
from tests.test_gpu_act_order_zp import _act_order_case, _int_zp_case

pytestmark = pytest.mark.gpu

TOL = 1e-2
GROUPS = {"u4b8": (-1, 32, 64, 128, 256), "u4": (-1, 32, 64, 128), "u8b128": (-1, 32, 128),
          "u8": (-1, 64, 128), "fp8": (-1, 128), "mxfp4": (32,), "nvfp4": (16,)}


def _case(i):
    rng = random.Random(9000 + i)
    fmt = FORMATS[i % len(FORMATS)]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    gs = rng.choice(GROUPS[fmt])
    unit = max(gs, 32) if gs > 0 else 32
    k = unit * rng.randint(1, 3072 // unit)
    n = 64 * rng.randint(1, 32)
    m = max(1, int(round(2 ** rng.uniform(0, math.log2(700)))))
    bias = rng.random() < 0.33
    return fmt, dtype, gs, m, n, k, bias


CASES = [_case(i) for i in range(112)]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_gemm_random_shapes(i):
    fmt, dtype, gs, m, n, k, bias = CASES[i]
    print(f"case sweep {i}: fmt={fmt} dtype={dtype} gs={gs} m={m} n={n} k={k} bias={bias}",
          flush=True)
    case = make_case(fmt, k, n, dtype, gs=gs, seed=500 + i)
    gen = torch.Generator().manual_seed(600 + i)
    a = torch.randn((m, k), generator=gen).to(dtype)
    b = torch.randn((n,), generator=gen).to(dtype) if bias else None
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, BITS[fmt])
    out = capi.marlin_gemm(a.cuda(), words, d.scales, case.type_id, m, n, k,
                           b_bias=O.marlin_permute_bias(b).cuda() if bias else None,
                           global_scale=d.global_scale, b_zeros=d.zeros,
                           is_zp_float=d.zeros is not None).cpu()
    assert O.max_abs_rel_err(out, O.gemm_ref(a, case.deq, b)) <= TOL


def _mode_case(i):
    rng = random.Random(9500 + i)
    mode = "act_order" if i % 2 else "int_zp"
    fmt = rng.choice(("u4b8", "u4", "u8b128") if mode == "act_order" else ("u4", "u8"))
    dtype = rng.choice([torch.float16, torch.bfloat16])
    gs = rng.choice((-1, 64, 128) if mode == "act_order" else (-1, 32, 64, 128))
    unit = max(gs, 32) if gs > 0 else 32
    k = unit * rng.randint(2, 2048 // unit)
    n = 64 * rng.randint(1, 24)
    m = max(1, int(round(2 ** rng.uniform(0, math.log2(500)))))
    return mode, fmt, dtype, gs, m, n, k


MODE_CASES = [_mode_case(i) for i in range(40)]


@pytest.mark.parametrize("i", range(len(MODE_CASES)))
def test_gemm_random_shapes_int_zero_points_and_act_order(i):
    """Random shapes for the two modes upstream marlin takes and the SM70 reference rejects:
    packed integer zero points (the oracle's single rounding of (q - z) * s) and act-order
    (weights repacked with perm = argsort(g_idx), every row scaled by its own group)."""
    mode, fmt, dtype, gs, m, n, k = MODE_CASES[i]
    print(f"case sweep-mode {i}: {mode} fmt={fmt} dtype={dtype} gs={gs} m={m} n={n} k={k}",
          flush=True)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(700 + i)).to(dtype)
    bits = BITS[fmt]
    if mode == "int_zp":
        q, s, z, _ = _int_zp_case(fmt, k, n, gs, dtype, seed=710 + i)
        words = capi.gptq_marlin_repack(O.gptq_pack(q, bits).cuda(), None, k, n, bits)
        out = capi.marlin_gemm(a.cuda(), words, s.cuda(), TYPE_ID[fmt], m, n, k,
                               b_zeros=O.pack_cols(z, bits).cuda(), is_zp_float=False).cpu()
        ref = O.gemm_ref(a, O.dequant_int_zero(q, s, z, dtype))
    else:
        g_idx, q, s, zp_f, deq = _act_order_case(fmt, k, n, gs, dtype, seed=720 + i)
        g_sorted, perm = marlin_sort_g_idx(g_idx)
        words = capi.gptq_marlin_repack(O.gptq_pack(q, bits).cuda(), perm.cuda(), k, n, bits)
        out = capi.marlin_gemm(a.cuda(), words, s.cuda(), TYPE_ID[fmt], m, n, k,
                               b_zeros=None if zp_f is None else zp_f.cuda(),
                               is_zp_float=zp_f is not None, g_idx=g_sorted.cuda(),
                               perm=perm.cuda()).cpu()
        ref = O.gemm_ref(a, deq)
    assert O.max_abs_rel_err(out, ref) <= TOL



def _large_case(i):
    rng = random.Random(9800 + i)
    fmt = FORMATS[(3 * i) % len(FORMATS)]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    gs = rng.choice(GROUPS[fmt])
    k = 128 * rng.randint(8, 64)
    n = 256 * rng.randint(8, 64)
    while n * k > (24 << 20) and k > 1024:  # keeps the oracle's quantizer to a few seconds
        k -= 128
    m = max(1, int(round(2 ** rng.uniform(0, 8))))
    return fmt, dtype, gs, m, n, k


LARGE_CASES = [_large_case(i) for i in range(12)]


@pytest.mark.parametrize("i", range(len(LARGE_CASES)))
def test_gemm_random_large_shapes(i):
    """Larger random shapes (N 2048-16384, K 1024-8192, M 1-256): the wide-N decode instances,
    the split mix of whole column groups and K-split leftovers, XCD-grouped block orders and
    the 128-row blocks at their production sizes."""
    fmt, dtype, gs, m, n, k = LARGE_CASES[i]
    print(f"case sweep-large {i}: fmt={fmt} dtype={dtype} gs={gs} m={m} n={n} k={k}", flush=True)
    case = make_case(fmt, k, n, dtype, gs=gs, seed=900 + i)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(950 + i)).to(dtype)
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, BITS[fmt])
    out = capi.marlin_gemm(a.cuda(), words, d.scales, case.type_id, m, n, k,
                           global_scale=d.global_scale, b_zeros=d.zeros,
                           is_zp_float=d.zeros is not None).cpu()
    assert O.max_abs_rel_err(out, O.gemm_ref(a, case.deq)) <= TOL
