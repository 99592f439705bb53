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
from tests.quant_cases import BITS, FORMATS, make_case, to_dev

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


CASES = [_case(i) for i in range(56)]


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
