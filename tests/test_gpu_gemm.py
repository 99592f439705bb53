"""GPU parity of marlin_gemm against the oracle (dequantize, fp32 matmul):
max|out - ref| <= 1e-2 * max|ref| for every format, both dtypes, small and large M (the
selector's 16/32/64/128-row tiles), split-K and K tails, bias, the strided-A path, and the
BASELINE configurations at full size."""
import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from tests.quant_cases import BITS, FORMATS, make_case, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max-abs error relative to max|ref|


def _run(case, a, bias=None, c=None):
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, case.k, case.n, BITS[case.fmt])
    return capi.marlin_gemm(a, words, d.scales, case.type_id, a.shape[0], case.n, case.k,
                            b_bias=bias, global_scale=d.global_scale, b_zeros=d.zeros,
                            is_zp_float=d.zeros is not None, c=c)


def _ref(case, a, bias_logical=None):
    return O.gemm_ref(a.cpu(), case.deq, bias_logical)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 16, 37, 64, 200])
def test_gemm_formats(fmt, dtype, m):
    k, n = 1024, 512
    print(f"case fmt={fmt} dtype={dtype} m={m} k={k} n={n}", flush=True)
    case = make_case(fmt, k, n, dtype, seed=m)
    gen = torch.Generator().manual_seed(100 + m)
    a = torch.randn((m, k), generator=gen).to(dtype)
    out = _run(case, a.cuda()).cpu()
    err = O.max_abs_rel_err(out, _ref(case, a))
    assert err <= TOL, err


@pytest.mark.parametrize("fmt", ["u4b8", "u4", "u8b128", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("k", [32, 96, 160, 4096 + 64])
def test_gemm_k_tail(fmt, k):
    n = 256
    if fmt in ("u4", "u4b8") and k % 128:
        gs = 32
    else:
        gs = None
    case = make_case(fmt, k, n, torch.bfloat16, gs=gs if (fmt in ("u4", "u4b8")) else None, seed=k)
    if case.gs not in (-1,) and k % case.gs:
        pytest.skip("group size does not divide K")
    a = torch.randn((16, k), generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
    print(f"case fmt={fmt} k={k}", flush=True)
    if fmt == "mxfp4" and k == 32:
        # one scale row reads as channelwise (group_size -1), which MXFP4 rejects, as the
        # reference does (marlin.cu:266-282, 479-493)
        with pytest.raises(capi.MarlinError, match="group_size 32"):
            _run(case, a.cuda())
        return
    out = _run(case, a.cuda()).cpu()
    assert O.max_abs_rel_err(out, _ref(case, a)) <= TOL


@pytest.mark.parametrize("gs", [-1, 32, 64, 128, 256])
def test_gemm_group_sizes(gs):
    k, n = 1024, 256
    case = make_case("u4", k, n, torch.float16, gs=gs, seed=gs + 1000)
    a = torch.randn((8, k), generator=torch.Generator().manual_seed(1)).half()
    out = _run(case, a.cuda()).cpu()
    assert O.max_abs_rel_err(out, _ref(case, a)) <= TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_bias_and_preallocated_c(dtype):
    k, n, m = 512, 256, 20
    case = make_case("u4b8", k, n, dtype, seed=5)
    gen = torch.Generator().manual_seed(6)
    a = torch.randn((m, k), generator=gen).to(dtype)
    bias = torch.randn((n,), generator=gen).to(dtype)
    c = torch.full((m, n), 7.0, dtype=dtype, device="cuda")
    out = _run(case, a.cuda(), bias=O.marlin_permute_bias(bias).cuda(), c=c)
    assert out.data_ptr() == c.data_ptr()
    assert O.max_abs_rel_err(out.cpu(), _ref(case, a, bias)) <= TOL


def test_gemm_strided_a():
    k, n, m = 512, 128, 9
    case = make_case("u4", k, n, torch.bfloat16, seed=9)
    big = torch.randn((m, k + 64), generator=torch.Generator().manual_seed(9)).bfloat16()
    a = big[:, 32:32 + k]
    out = _run(case, big.cuda()[:, 32:32 + k]).cpu()
    assert O.max_abs_rel_err(out, _ref(case, a)) <= TOL


def test_gemm_split_k_repeatable():
    # split-K workspace must be left zeroed: repeated calls give identical results
    k, n, m = 8192, 256, 4
    case = make_case("u4b8", k, n, torch.float16, seed=11)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(2)).half().cuda()
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, 4)
    outs = [capi.marlin_gemm(a, words, d.scales, case.type_id, m, n, k) for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) or O.max_abs_rel_err(outs[0].cpu(), outs[1].cpu()) < 1e-3
    assert O.max_abs_rel_err(outs[2].cpu(), _ref(case, a.cpu())) <= TOL


def test_gemm_m_zero():
    k, n = 256, 128
    case = make_case("u4b8", k, n, torch.float16, seed=1)
    a = torch.empty((0, k), dtype=torch.float16, device="cuda")
    out = _run(case, a)
    assert out.shape == (0, n)


# BASELINE shapes at full size (the selector's production paths: the headline decode kernel
# with its whole-group / K-split block mix, the multistage and 128-row kernels); rows of
# large-M outputs are checked on a fixed sample spread over M.
BASELINE_SHAPES = [
    ("cfg1", "u4b8", torch.float16, 16, 4096, 4096),
    ("cfg2", "u4", torch.bfloat16, 1, 5120, 34816),
    ("cfg2", "u4", torch.bfloat16, 16, 5120, 34816),
    ("cfg2", "u4", torch.bfloat16, 128, 5120, 34816),
    ("cfg2", "u4", torch.bfloat16, 1024, 5120, 34816),
    ("cfg3", "u8b128", torch.float16, 4096, 8192, 8192),
    ("cfg4", "mxfp4", torch.bfloat16, 1, 3072, 12288),
    ("cfg4", "mxfp4", torch.bfloat16, 512, 3072, 12288),
    ("cfg4", "nvfp4", torch.bfloat16, 1, 3072, 12288),
    ("cfg4", "nvfp4", torch.bfloat16, 64, 3072, 12288),
]


@pytest.mark.parametrize("name,fmt,dtype,m,k,n", BASELINE_SHAPES)
def test_gemm_baseline_shapes(name, fmt, dtype, m, k, n):
    print(f"case {name} fmt={fmt} m={m} k={k} n={n}", flush=True)
    case = make_case(fmt, k, n, dtype, seed=m + k)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(m)).to(dtype)
    out = _run(case, a.cuda()).cpu()
    rows = torch.arange(m) if m <= 64 else torch.unique(torch.linspace(0, m - 1, 64).long())
    ref = O.gemm_ref(a[rows], case.deq)
    assert O.max_abs_rel_err(out[rows], ref) <= TOL
