"""marlin_gemm_no_alloc (the entry point that allocates nothing: split-K scratch in a static
per-GPU device array) against marlin_gemm on the same inputs, through the C ABI: two calls
in a row, the second smaller, each within the GEMM tolerance of marlin_gemm's output and of
the oracle; a shape whose split-K plan needs more scratch than the array holds is rejected."""
import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from tests.quant_cases import BITS, make_case, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _both(case, m, seed):
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, case.k, case.n, BITS[case.fmt])
    a = torch.randn((m, case.k), generator=torch.Generator().manual_seed(seed)).to(case.dtype)
    a = a.cuda()
    kw = dict(global_scale=d.global_scale, b_zeros=d.zeros, is_zp_float=d.zeros is not None)
    ref = capi.marlin_gemm(a, words, d.scales, case.type_id, m, case.n, case.k, **kw)
    got = capi.marlin_gemm_no_alloc(a, words, d.scales, case.type_id, m, case.n, case.k, **kw)
    torch.cuda.synchronize()
    return a.cpu(), ref.cpu(), got.cpu()


@pytest.mark.parametrize("fmt,dtype", [("u4b8", torch.float16), ("u4", torch.bfloat16),
                                       ("nvfp4", torch.bfloat16)])
def test_no_alloc_matches_marlin_gemm_twice(fmt, dtype):
    # first: a 64-row multistage block over K = 8192 (split K 16 ways); second, smaller: a
    # decode shape whose 16-column groups split K across workgroups
    for m, k, n, seed in ((64, 8192, 512, 1), (4, 4096, 256, 2)):
        print(f"case no-alloc fmt={fmt} dtype={dtype} m={m} k={k} n={n}", flush=True)
        case = make_case(fmt, k, n, dtype, seed=seed + 31)
        a, ref, got = _both(case, m, seed)
        assert O.max_abs_rel_err(got, ref) <= TOL
        assert O.max_abs_rel_err(got, O.gemm_ref(a, case.deq)) <= TOL


def test_no_alloc_large_m_then_repeat():
    # a 300-row call on 128-row blocks, then one decode shape three times: the scratch the
    # earlier calls used must read as zero again
    case = make_case("u8b128", 1024, 512, torch.float16, seed=5)
    a, ref, got = _both(case, 300, 7)
    assert O.max_abs_rel_err(got, ref) <= TOL
    case = make_case("u4b8", 8192, 256, torch.float16, seed=11)
    for i in range(3):
        a, ref, got = _both(case, 4, 2)
        assert O.max_abs_rel_err(got, ref) <= TOL, i


def test_no_alloc_rejects_scratch_beyond_limit():
    # M = 1280, N = 2048, K = 1024, uint4b8 in 32-deep groups: beyond 1024 rows small groups
    # take the tiled kernel, whose 10 x 8 blocks of 128 x 256 on 256 CUs split K in two and
    # need M * N = 2.6M partial sums, above the 2M the static scratch holds
    m, k, n = 1280, 1024, 2048
    case = make_case("u4b8", k, n, torch.float16, gs=32, seed=3)
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, 4)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(4)).half().cuda()
    with pytest.raises(capi.MarlinError, match="static scratch holds 2097152"):
        capi.marlin_gemm_no_alloc(a, words, d.scales, case.type_id, m, n, k)
    # the regular entry point runs the same shape
    out = capi.marlin_gemm(a, words, d.scales, case.type_id, m, n, k)
    rows = torch.arange(0, m, 37)
    assert O.max_abs_rel_err(out.cpu()[rows], O.gemm_ref(a.cpu()[rows], case.deq)) <= TOL
