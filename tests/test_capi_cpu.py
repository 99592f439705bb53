"""CPU checks of the C ABI: the library loads, exports every function include/*.h declares,
and rejects invalid arguments before touching a GPU (the reference's TORCH_CHECK
contract, csrc/quantization/marlin/marlin.cu:95-383, csrc/moe/marlin_moe_wna16/ops.cu:118-402)."""
import ctypes
import os
import re

import pytest

from marlin_v100_amd import capi
from tests.quant_cases import TYPE_ID

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            text = open(os.path.join(inc, f)).read()
            names |= set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(marlin_\w+)\s*\(", text, re.M))
    return names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(capi.LIB_PATH)
    declared = _declared_symbols()
    assert {"marlin_gemm", "marlin_moe_wna16_marlin_gemm", "marlin_moe_align_block_size",
            "marlin_gptq_marlin_repack", "marlin_awq_marlin_repack"} <= declared
    for name in declared:
        assert hasattr(lib, name), name
    assert set(capi.SIGNATURES) == declared


def test_abi_version():
    assert capi.load().marlin_abi_version() == 2


def _gemm(**kw):
    args = dict(a=16, a_dtype=capi.F16, a_row_stride=256, c=16, bq=16, bq_numel=256 * 512 // 8,
                bias=None, bias_numel=0, scales=16, scales_dtype=capi.F16, scales_numel=2 * 512,
                groups=2, a_scales_numel=0, glob=None, glob_numel=0, zeros=None,
                zeros_dtype=capi.F16, zeros_numel=0, gidx_ptr=None, gidx=0, perm_ptr=None, perm=0,
                type_id=TYPE_ID["u4b8"], m=4, n=512, k=256, zp_float=0, k_full=1)
    args.update(kw)
    lib = capi.load()
    st = lib.marlin_gemm(args["a"], args["a_dtype"], args["a_row_stride"], args["c"], args["bq"],
                         args["bq_numel"], args["bias"], args["bias_numel"], args["scales"],
                         args["scales_dtype"], args["scales_numel"], args["groups"],
                         args["a_scales_numel"], args["glob"], args["glob_numel"], args["zeros"],
                         args["zeros_dtype"], args["zeros_numel"], args["gidx_ptr"], args["gidx"],
                         args["perm_ptr"], args["perm"], None, 0, args["type_id"], args["m"],
                         args["n"], args["k"], args["k_full"], 0, 0, args["zp_float"], None)
    return st, lib.marlin_get_last_error().decode()


@pytest.mark.parametrize("kw,status,msg", [
    (dict(gidx=4), capi.STATUS_INVALID, "act_order needs g_idx and perm"),
    (dict(perm=256, perm_ptr=16), capi.STATUS_INVALID, "act_order needs g_idx and perm"),
    (dict(gidx=256, perm=256), capi.STATUS_INVALID, "null g_idx / perm"),
    (dict(gidx=256, perm=256, gidx_ptr=16, perm_ptr=16, k_full=0), capi.STATUS_NOT_SUPPORTED,
     "is_k_full=false"),
    (dict(gidx=256, perm=256, gidx_ptr=16, perm_ptr=16, type_id=TYPE_ID["fp8"],
          scales_dtype=capi.F16, groups=1, scales_numel=512), capi.STATUS_NOT_SUPPORTED,
     "integer weight types"),
    (dict(type_id=TYPE_ID["u4"], zeros=16, zeros_numel=2 * 512 // 8, zeros_dtype=capi.F16),
     capi.STATUS_INVALID, "must be int32"),
    (dict(type_id=TYPE_ID["u4"], zeros=16, zeros_numel=2 * 512, zeros_dtype=capi.I32),
     capi.STATUS_INVALID, "num_groups * size_n / pack_factor"),
    (dict(a_dtype=capi.F32), capi.STATUS_NOT_SUPPORTED, "float16 and bfloat16"),
    (dict(type_id=12345), capi.STATUS_NOT_SUPPORTED, "implements only"),
    (dict(n=96, scales_numel=2 * 96, bq_numel=256 * 96 // 8), capi.STATUS_INVALID,
     "size_n % 64 == 0"),
    (dict(k=240, a_row_stride=240, scales_numel=512, groups=1, bq_numel=240 * 512 // 8),
     capi.STATUS_INVALID, "size_k % 32 == 0"),
    (dict(zeros=16, zeros_numel=2 * 512, zp_float=1), capi.STATUS_INVALID, "zero-point"),
    (dict(type_id=TYPE_ID["u4"]), capi.STATUS_INVALID, "requires zero points"),
    (dict(zp_float=1), capi.STATUS_INVALID, "is_zp_float is true but b_zeros"),
    (dict(groups=3, scales_numel=3 * 512), capi.STATUS_INVALID, "not divisible by b_scales"),
    (dict(groups=16, scales_numel=16 * 512), capi.STATUS_INVALID, "unsupported group_size"),
    (dict(glob=16, glob_numel=1), capi.STATUS_INVALID, "global_scale is supported only"),
    (dict(type_id=TYPE_ID["nvfp4"], scales_dtype=capi.F8E4M3, groups=16,
          scales_numel=16 * 512), capi.STATUS_INVALID, "global_scale parameter must be passed"),
    (dict(type_id=TYPE_ID["nvfp4"], scales_dtype=capi.F16), capi.STATUS_INVALID,
     "float8_e4m3fn for NVFP4"),
    (dict(type_id=TYPE_ID["mxfp4"], scales_dtype=capi.F8E8M0), capi.STATUS_INVALID,
     "group_size 32"),
    (dict(scales_dtype=capi.BF16), capi.STATUS_INVALID, "activation dtype"),
    (dict(a_row_stride=250), capi.STATUS_INVALID, "stride(0) must divisible by 8"),
    (dict(a_scales_numel=4), capi.STATUS_INVALID, "a_scales"),
    (dict(bq_numel=5), capi.STATUS_INVALID, "b_q_weight numel"),
])
def test_gemm_rejections(kw, status, msg):
    st, err = _gemm(**kw)
    assert st == status, err
    assert msg in err, err


def test_no_alloc_rejects_act_order():
    lib = capi.load()
    st = lib.marlin_gemm_no_alloc(16, capi.F16, 256, 16, 16, 256 * 256 // 8, None, 0, 16,
                                  capi.F16, 2 * 256, 2, 0, None, 0, None, capi.F16, 0, 256, 256,
                                  TYPE_ID["u4b8"], 2, 256, 256, 0, None)
    assert st == capi.STATUS_NOT_SUPPORTED
    assert "act_order" in lib.marlin_get_last_error().decode()


def test_gemm_m_zero_is_noop():
    st, err = _gemm(m=0, a=None, c=None)
    assert st == capi.STATUS_OK, err


def test_repack_rejections():
    lib = capi.load()
    assert lib.marlin_gptq_marlin_repack(None, 0, None, 0, 100, 64, 4, 0, None, 0, None) == 1
    assert "tile_k_size" in lib.marlin_get_last_error().decode()
    assert lib.marlin_gptq_marlin_repack(None, 0, None, 0, 128, 64, 3, 0, None, 0, None) == 1
    assert "num_bits must be 4 or 8" in lib.marlin_get_last_error().decode()
    # the 8-bit-activation layout has no act-order form (gptq_marlin_repack.cu:377-396)
    assert lib.marlin_gptq_marlin_repack(None, 128 * 64 // 8, None, 128, 128, 64, 4, 1, None,
                                         128 * 64 // 8, None) == 1
    assert "Unsupported repack config" in lib.marlin_get_last_error().decode()
    # ... but is otherwise accepted (empty sizes: validated, nothing launched)
    assert lib.marlin_gptq_marlin_repack(None, 0, None, 0, 0, 64, 4, 1, None, 0, None) == 0
    assert lib.marlin_awq_marlin_repack(None, 0, 0, 64, 8, 1, None, 0, None) == 0
    assert lib.marlin_awq_marlin_repack(None, 5, 128, 64, 4, 0, None, 0, None) == 1
    assert "Shape mismatch" in lib.marlin_get_last_error().decode()


def test_int4_fp8_preprocess_rejections():
    """marlin_int4_fp8_preprocess.cu:60-92."""
    lib = capi.load()
    fake = ctypes.c_void_p(16)  # never dereferenced: every case fails validation first
    assert lib.marlin_int4_fp8_preprocess(fake, 3, 5, None, 0, 0, fake, None) == 1
    assert "% 256 != 0" in lib.marlin_get_last_error().decode()
    assert lib.marlin_int4_fp8_preprocess(fake, 48, 4, fake, 3, 4, fake, None) == 1
    assert "size_k % 32 != 0" in lib.marlin_get_last_error().decode()
    assert lib.marlin_int4_fp8_preprocess(fake, 64, 4, fake, 2, 8, fake, None) == 1
    assert "qweight.size(1) != qzeros.size(1)" in lib.marlin_get_last_error().decode()
    assert lib.marlin_int4_fp8_preprocess(fake, 64, 4, fake, 3, 4, fake, None) == 1
    assert "qweight.size(0) % qzeros.size(0) != 0" in lib.marlin_get_last_error().decode()
    assert lib.marlin_int4_fp8_preprocess(fake, 64, 4, fake, 16, 4, fake, None) == 1
    assert "group_size % 8 != 0" in lib.marlin_get_last_error().decode()
    assert lib.marlin_int4_fp8_preprocess(None, 0, 8, None, 0, 0, None, None) == 0


def test_moe_rejections():
    lib = capi.load()

    def call(bs=64, type_id=TYPE_ID["u4"], zeros_numel=8 * 2 * 512, zp=1):
        st = lib.marlin_moe_wna16_marlin_gemm(
            16, capi.BF16, 16, 16, 8 * 256 * 512 // 8, 8, None, 0, 16, capi.BF16, 8 * 2 * 512, 2,
            0, None, 0, 16, capi.BF16, zeros_numel, 0, 0, None, 0, 16, 100, 16, 10, 16, 16, 64,
            bs, 4, 0, type_id, 16, 512, 256, 1, 0, 0, zp, -1, -1, -1, None)
        return st, lib.marlin_get_last_error().decode()

    st, err = call(bs=24)
    assert st == 1 and "unsupported moe_block_size=24" in err
    st, err = call(bs=128)
    assert st == 1 and "unsupported moe_block_size=128" in err
    st, err = call(zeros_numel=0, zp=0)
    assert st == 1 and "requires zero points" in err


def test_moe_align_rejections():
    lib = capi.load()
    st = lib.marlin_moe_align_block_size(16, capi.I32, 8, 2000, 16, 16, 100, 16, 10, 16, None, 0,
                                         None)
    assert st == 1 and "padded_num_experts" in lib.marlin_get_last_error().decode()
    st = lib.marlin_moe_align_block_size(16, capi.F32, 8, 8, 16, 16, 100, 16, 10, 16, None, 0,
                                         None)
    assert st == 1 and "int32 or int64" in lib.marlin_get_last_error().decode()


def test_topk_router_rejections():
    lib = capi.load()

    def call(fn, ids_dt=capi.I32, k=2, g_dt=capi.F16, t=4, e=8, bias_numel=0):
        bias = 16 if bias_numel else None
        st = fn(16, 16, ids_dt, 16, k, 16, g_dt, t, e, 1, bias, bias_numel, None)
        return st, lib.marlin_get_last_error().decode()

    for fn in (lib.marlin_topk_softmax, lib.marlin_topk_sigmoid):
        st, err = call(fn, bias_numel=7)
        assert st == 1 and "bias size mismatch, expected: 8" in err
        st, err = call(fn, g_dt=capi.I32)
        assert st == 1 and "Unsupported gating_output data type" in err
        st, err = call(fn, ids_dt=capi.F32)
        assert st == 1 and "int32, uint32 or int64" in err
        st, err = call(fn, k=9)
        assert st == 1 and "topk" in err
        st, err = call(fn, e=8192, k=2)
        assert st == 2 and "experts" in err
        st, err = call(fn, e=1024, k=300)
        assert st == 2 and "topk <= 256" in err
        assert call(fn, t=0)[0] == 0  # no tokens: nothing to launch


def test_grouped_topk_rejections():
    lib = capi.load()

    def call(scores_dt=capi.F32, bias_dt=capi.F32, e=16, ng=4, tg=2, k=2, sf=0, bias_numel=16):
        st = lib.marlin_grouped_topk(16, scores_dt, 4, e, ng, tg, k, 1, 1.0, 16, bias_dt,
                                     bias_numel, sf, 16, 16, None)
        return st, lib.marlin_get_last_error().decode()

    assert call(scores_dt=capi.I32)[1].startswith("Invalid dtype")
    assert call(bias_dt=capi.I64)[1].startswith("Invalid bias dtype")
    assert "divisible by n_group" in call(e=18, bias_numel=18)[1]
    assert "topk_group must be <= n_group" in call(tg=5)[1]
    assert "n_group should be smaller than or equal to 32" in call(e=64, ng=64, bias_numel=64)[1]
    assert "topk should be smaller than or equal to 32" in call(e=256, k=33, bias_numel=256)[1]
    assert "topk must be <= topk_group" in call(k=9)[1]
    assert "scoring_func must be" in call(sf=2)[1]
    assert "bias size mismatch" in call(bias_numel=15)[1]
    st, err = call(e=2048, bias_numel=2048)
    assert st == 2 and "1024" in err


def test_moe_align_buffer_size_rejections():
    """A sorted_token_ids buffer shorter than numel + E * (bs - 1) would drop routes: it is
    rejected before any launch (the reference sizes it so, moe_align_block_size.py:15)."""
    lib = capi.load()
    # numel 8, E 4, bs 16 -> needs 8 + 4 * 15 = 68 slots and ceil(68 / 16) = 5 expert ids
    st = lib.marlin_moe_align_block_size(16, capi.I32, 8, 4, 16, 16, 67, 16, 5, 16, None, 0, None)
    err = lib.marlin_get_last_error().decode()
    assert st == 1 and "sorted_token_ids must hold" in err and "68" in err, err
    st = lib.marlin_moe_align_block_size(16, capi.I32, 8, 4, 16, 16, 68, 16, 4, 16, None, 0, None)
    err = lib.marlin_get_last_error().decode()
    assert st == 1 and "experts_ids must hold" in err, err


def test_moe_sum_dtypes():
    lib = capi.load()
    assert lib.marlin_moe_sum(16, capi.I32, 4, 2, 8, 16, None) == 1
    assert "float16, bfloat16 and float32" in lib.marlin_get_last_error().decode()
    # fp32 is accepted, and there is no token limit (nothing to launch at hidden 0)
    assert lib.marlin_moe_sum(16, capi.F32, 1 << 20, 8, 0, 16, None) == 0


def test_moe_size_n_multiple_of_64_is_accepted():
    """size_n % 64 == 0 passes validation (reference ops.cu:390-392); without a GPU the call
    then stops at the device query, not at a NOT_SUPPORTED size check."""
    lib = capi.load()
    e, n, k = 8, 320, 256
    st = lib.marlin_moe_wna16_marlin_gemm(
        16, capi.BF16, 16, 16, e * k * n // 8, e, None, 0, 16, capi.BF16, e * 2 * n, 2,
        0, None, 0, 16, capi.BF16, e * 2 * n, 0, 0, None, 0, 16, 100, 16, 10, 16, 16, 64,
        16, 4, 0, TYPE_ID["u4"], 16, n, k, 1, 0, 0, 1, -1, -1, -1, None)
    err = lib.marlin_get_last_error().decode()
    assert st != capi.STATUS_NOT_SUPPORTED and "256" not in err, (st, err)
    st = lib.marlin_moe_wna16_marlin_gemm(
        16, capi.BF16, 16, 16, e * k * 96 // 8, e, None, 0, 16, capi.BF16, e * 2 * 96, 2,
        0, None, 0, 16, capi.BF16, e * 2 * 96, 0, 0, None, 0, 16, 100, 16, 10, 16, 16, 64,
        16, 4, 0, TYPE_ID["u4"], 16, 96, k, 1, 0, 0, 1, -1, -1, -1, None)
    assert st == 1 and "min_thread_n" in lib.marlin_get_last_error().decode()


def test_product_scalar_type_round_trips_ids():
    from marlin_v100_amd.scalar_type import NanRepr, ScalarType, scalar_types

    for name in ("uint4", "uint4b8", "uint8", "uint8b128", "float4_e2m1f", "float8_e4m3fn",
                 "float8_e8m0fnu"):
        t = getattr(scalar_types, name)
        assert ScalarType.from_id(t.id) == t and str(t) == name
    odd = ScalarType(3, 2, True, 5, False, NanRepr.IEEE_754)
    assert ScalarType.from_id(odd.id) == odd
    with pytest.raises(ValueError):
        ScalarType.from_id(-1)
    with pytest.raises(ValueError):
        ScalarType.from_id(1 << 60)
