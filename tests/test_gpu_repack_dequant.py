"""GPU parity: repack (GPTQ and AWQ sources) followed by the device dequant routines the
GEMM uses must reproduce the oracle's dequantized weights bit-exactly, for every format,
both activation dtypes, and K with and without a partial 128-deep tail."""
import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from tests.quant_cases import FORMATS, make_case, to_dev

pytestmark = pytest.mark.gpu

SHAPES = [(128, 64), (256, 192), (160, 64), (96, 128), (4096, 256)]


def _dequant(case, words):
    return capi.dequantize(words, case.scales, case.type_id, case.k, case.n, case.dtype,
                           b_zeros=case.zeros, global_scale=case.global_scale)


def _gs_for(fmt, k):
    from tests.quant_cases import DEFAULT_GS
    gs = DEFAULT_GS[fmt]
    if gs != -1 and k % gs:
        gs = {"fp8": -1}.get(fmt, 32)
    return gs


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k,n", SHAPES)
def test_gptq_repack_dequant_bit_exact(fmt, dtype, k, n):
    case = make_case(fmt, k, n, dtype, gs=_gs_for(fmt, k), seed=k + n)
    print(f"case fmt={fmt} dtype={dtype} k={k} n={n}", flush=True)
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, 8 if fmt in ("u8b128", "u8", "fp8") else 4)
    out = _dequant(d, words).cpu()
    bad = (out.view(torch.int16) != case.deq.view(torch.int16)).nonzero()[:5]
    assert bad.numel() == 0, (
        f"mismatch at {bad.tolist()}: got bits "
        f"{[hex(int(out.view(torch.int16)[i, j]) & 0xffff) for i, j in bad.tolist()]} want "
        f"{[hex(int(case.deq.view(torch.int16)[i, j]) & 0xffff) for i, j in bad.tolist()]}")


@pytest.mark.parametrize("fmt", ["u4b8", "u4", "u8b128", "u8"])
@pytest.mark.parametrize("k,n", [(128, 64), (160, 128), (256, 256)])
def test_awq_repack_matches_gptq_repack(fmt, k, n):
    case = make_case(fmt, k, n, torch.float16, seed=7)
    d = to_dev(case)
    bits = 4 if fmt.startswith("u4") else 8
    a = capi.awq_marlin_repack(d.awq_words, k, n, bits)
    g = capi.gptq_marlin_repack(d.gptq_words, None, k, n, bits)
    assert torch.equal(a, g)


@pytest.mark.parametrize("bits", [4, 8])
def test_gptq_repack_with_perm(bits):
    k, n = 256, 128
    gen = torch.Generator().manual_seed(3)
    q = torch.randint(0, 1 << bits, (k, n), generator=gen, dtype=torch.int32)
    perm = torch.randperm(k, generator=gen).to(torch.int32)
    # repack(pack(q), perm) must equal repack(pack(q[perm])) (act-order row gather)
    words = O.gptq_pack(q, bits).cuda()
    with_perm = capi.gptq_marlin_repack(words, perm.cuda(), k, n, bits)
    plain = capi.gptq_marlin_repack(O.gptq_pack(q[perm.long()], bits).cuda(), None, k, n, bits)
    assert torch.equal(with_perm, plain)


def test_repack_is_a_permutation_of_words():
    k, n = 512, 256
    words = torch.arange(k // 8 * n, dtype=torch.int32).reshape(k // 8, n).cuda()
    out = capi.gptq_marlin_repack(words, None, k, n, 4)
    assert out.shape == (k // 16, n * 2)
    assert torch.equal(out.flatten().sort().values, words.flatten().sort().values)
