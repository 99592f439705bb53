"""Seeded random sweep of the repack ops: gptq_marlin_repack followed by the device dequant
reproduces the oracle's dequantized weights bit for bit (every format, both dtypes, the group
sizes each format allows, K any multiple of the group size and of 32, N any multiple of 64);
awq_marlin_repack of the AWQ packing equals the GPTQ repack; a repack with an act-order perm
equals the plain repack of the row-gathered codes."""
import random

import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from tests.quant_cases import BITS, FORMATS, make_case, to_dev

pytestmark = pytest.mark.gpu

GROUPS = {"u4b8": (-1, 32, 64, 128), "u4": (32, 64, 128), "u8b128": (-1, 64, 128),
          "u8": (64, 128), "fp8": (-1, 128), "mxfp4": (32,), "nvfp4": (16,)}


def _case(i):
    rng = random.Random(6000 + i)
    fmt = FORMATS[i % len(FORMATS)]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    gs = rng.choice(GROUPS[fmt])
    unit = max(gs, 32)  # the gfx950 layout takes size_k % 32 (the reference: % 16)
    k = unit * rng.randint(1, 2048 // unit)
    n = 64 * rng.randint(1, 64)
    return fmt, dtype, gs, k, n


CASES = [_case(i) for i in range(42)]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_repack_dequant_random_shapes(i):
    fmt, dtype, gs, k, n = CASES[i]
    print(f"case repack-sweep {i}: fmt={fmt} dtype={dtype} gs={gs} k={k} n={n}", flush=True)
    case = make_case(fmt, k, n, dtype, gs=gs, seed=300 + i)
    d = to_dev(case)
    bits = BITS[fmt]
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, bits)
    out = capi.dequantize(words, d.scales, case.type_id, k, n, dtype, b_zeros=d.zeros,
                          global_scale=d.global_scale).cpu()
    assert torch.equal(out.view(torch.int16), case.deq.view(torch.int16))
    if d.awq_words is not None:
        assert torch.equal(capi.awq_marlin_repack(d.awq_words, k, n, bits), words)


@pytest.mark.parametrize("i", range(12))
def test_repack_perm_random_shapes(i):
    rng = random.Random(6500 + i)
    bits = rng.choice([4, 8])
    k = 32 * rng.randint(1, 64)
    n = 64 * rng.randint(1, 32)
    print(f"case repack-perm-sweep {i}: bits={bits} k={k} n={n}", flush=True)
    gen = torch.Generator().manual_seed(6600 + i)
    q = torch.randint(0, 1 << bits, (k, n), generator=gen, dtype=torch.int32)
    perm = torch.randperm(k, generator=gen).to(torch.int32)
    with_perm = capi.gptq_marlin_repack(O.gptq_pack(q, bits).cuda(), perm.cuda(), k, n, bits)
    plain = capi.gptq_marlin_repack(O.gptq_pack(q[perm.long()], bits).cuda(), None, k, n, bits)
    assert torch.equal(with_perm, plain)
