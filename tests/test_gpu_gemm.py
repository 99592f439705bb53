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
    ("cfg4", "mxfp4", torch.bfloat16, 64, 3072, 12288),
    ("cfg4", "mxfp4", torch.bfloat16, 512, 3072, 12288),
    ("cfg4", "nvfp4", torch.bfloat16, 1, 3072, 12288),
    ("cfg4", "nvfp4", torch.bfloat16, 64, 3072, 12288),
    ("cfg4", "nvfp4", torch.bfloat16, 512, 3072, 12288),
    # a partial 128-row block (65..128 rows on wide N) and ragged 64-row fp4 blocks
    ("cfg2", "u4", torch.bfloat16, 80, 5120, 34816),
    ("cfg4", "nvfp4", torch.bfloat16, 1000, 3072, 12288),
    ("cfg4", "mxfp4", torch.bfloat16, 777, 3072, 12288),
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


# The tiled kernel (marlin_gemm_kernel) serves what the other two do not instantiate: M > 128
# with N % 256 != 0 (16-row x 64-column tiles, split K when the grid is small) and groups
# below 128 beyond M = 1024 (fp4 weights: beyond M = 2048; 128 x 256 tiles).  K = 1056 leaves
# a 32-deep tail after the 256-deep steps.
TILED_CASES = [(fmt, dt, m, n, k) for fmt in ("u4b8", "u4", "u8b128", "fp8")
               for dt in (torch.float16, torch.bfloat16)
               for m, n, k in ((129, 192, 1024), (200, 320, 1024))]
TILED_CASES += [("u8b128", torch.float16, 200, 320, 1056), ("u8b128", torch.bfloat16, 1500, 384, 1056)]


@pytest.mark.parametrize("fmt,dtype,m,n,k", TILED_CASES)
def test_gemm_tiled_kernel_narrow_n(fmt, dtype, m, n, k):
    print(f"case tiled fmt={fmt} dtype={dtype} m={m} n={n} k={k}", flush=True)
    case = make_case(fmt, k, n, dtype, seed=m + n + k)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(m + n)).to(dtype)
    out = _run(case, a.cuda()).cpu()
    assert O.max_abs_rel_err(out, _ref(case, a)) <= TOL


@pytest.mark.parametrize("fmt,gs", [("u4", 32), ("u4b8", 64), ("mxfp4", None), ("nvfp4", None)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_tiled_kernel_small_groups_large_m(fmt, gs, dtype):
    m, k, n = (2100 if fmt in ("mxfp4", "nvfp4") else 1100), 1024, 512
    print(f"case tiled-small-group fmt={fmt} gs={gs} dtype={dtype} m={m}", flush=True)
    case = make_case(fmt, k, n, dtype, gs=gs, seed=77)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(78)).to(dtype)
    out = _run(case, a.cuda()).cpu()
    rows = torch.unique(torch.linspace(0, m - 1, 96).long())
    assert O.max_abs_rel_err(out[rows], O.gemm_ref(a[rows], case.deq)) <= TOL


_WIDE_CASES = {}


def _wide_case(fmt, dtype):
    key = (fmt, dtype)
    if key not in _WIDE_CASES:
        _WIDE_CASES[key] = make_case(fmt, 1024, 16384, dtype, seed=4242)
    return _WIDE_CASES[key]


@pytest.mark.parametrize("fmt", ["u4b8", "u4", "u8b128", "u8", "fp8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [2, 4, 8])
def test_gemm_decode_wide_n(fmt, dtype, m):
    """N = 16384: more 64-column groups than CUs, the decode kernel's three-waves-per-SIMD
    instances (two steps in flight up to eight rows, or its depth-3 fallback)."""
    print(f"case wide-n fmt={fmt} dtype={dtype} m={m}", flush=True)
    case = _wide_case(fmt, dtype)
    a = torch.randn((m, case.k), generator=torch.Generator().manual_seed(m)).to(dtype)
    out = _run(case, a.cuda()).cpu()
    assert O.max_abs_rel_err(out, _ref(case, a)) <= TOL


def test_gemm_graph_capture_on_side_stream():
    """A split-K shape captured into a HIP graph on a side stream after one eager call on
    that stream: every replay (with eager work and syncs between) equals the eager output.
    Capturing a shape whose workspace was never sized on the capturing stream is a clean
    error, not an allocation inside the capture."""
    k, n, m = 8192, 256, 4
    case = make_case("u4b8", k, n, torch.float16, seed=11)
    d = to_dev(case)
    words = capi.gptq_marlin_repack(d.gptq_words, None, k, n, 4)
    a = torch.randn((m, k), generator=torch.Generator().manual_seed(3)).half().cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = capi.marlin_gemm(a, words, d.scales, case.type_id, m, n, k)
        c = torch.empty_like(eager)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            capi.marlin_gemm(a, words, d.scales, case.type_id, m, n, k, c=c)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref = eager.cpu()
    for i in range(4):
        c.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        other = capi.marlin_gemm(a, words, d.scales, case.type_id, m, n, k)  # eager work between
        torch.cuda.synchronize()
        assert O.max_abs_rel_err(c.cpu(), ref) <= 1e-3, i
        assert O.max_abs_rel_err(other.cpu(), ref) <= 1e-3, i
    assert O.max_abs_rel_err(ref, _ref(case, a.cpu())) <= TOL

    # a fresh stream has no workspace: capture must fail cleanly
    fresh = torch.cuda.Stream()
    fresh.wait_stream(torch.cuda.current_stream())
    g2 = torch.cuda.CUDAGraph()
    with pytest.raises(capi.MarlinError, match="capturing stream"):
        with torch.cuda.graph(g2, stream=fresh):
            capi.marlin_gemm(a, words, d.scales, case.type_id, m, n, k, c=c)
    torch.cuda.synchronize()
