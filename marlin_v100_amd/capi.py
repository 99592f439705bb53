"""ctypes binding of libmarlin_mi355x.so (the C ABI in include/marlin_mi355x.h).

This is the binding a maintainer of a ctypes/FFI caller would write; the GPU parity tests
call the kernels through it.  Tensors here are torch tensors used only as device memory.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmarlin_mi355x.so")

# marlin_dtype_t
F16, BF16, F32, F8E4M3, F8E8M0, I32, I64, U8, I8, U32 = range(10)
_DT = {
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.float32: F32,
    torch.float8_e4m3fn: F8E4M3,
    torch.float8_e8m0fnu: F8E8M0,
    torch.int32: I32,
    torch.int64: I64,
    torch.uint8: U8,
    torch.int8: I8,
    torch.uint32: U32,
}

STATUS_OK, STATUS_INVALID, STATUS_NOT_SUPPORTED, STATUS_HIP = range(4)

# Every exported symbol and its ctypes signature.
_P, _I64, _I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "marlin_get_last_error": (ctypes.c_char_p, []),
    "marlin_abi_version": (_I, []),
    "marlin_gptq_marlin_repack": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P]),
    "marlin_awq_marlin_repack": (_I, [_P, _I64, _I64, _I64, _I64, _I, _P, _I64, _P]),
    "marlin_int4_fp8_preprocess": (_I, [_P, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "marlin_gemm": (_I, [_P, _I, _I64, _P, _P, _I64, _P, _I64, _P, _I, _I64, _I64, _I64, _P, _I64,
                         _P, _I, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I,
                         _I, _I, _I, _P]),
    "marlin_gemm_no_alloc": (_I, [_P, _I, _I64, _P, _P, _I64, _P, _I64, _P, _I, _I64, _I64,
                                  _I64, _P, _I64, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64,
                                  _I64, _I, _P]),
    "marlin_moe_align_block_size": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P,
                                         _I64, _P]),
    "marlin_moe_wna16_marlin_gemm": (_I, [_P, _I, _P, _P, _I64, _I64, _P, _I64, _P, _I, _I64,
                                          _I64, _I64, _P, _I64, _P, _I, _I64, _I64, _I64, _P,
                                          _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I,
                                          _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I64, _I64,
                                          _I64, _P]),
    "marlin_moe_wna16_marlin_gemm_silu": (_I, [_P, _I, _P, _P, _I64, _I64, _P, _I64, _P, _I,
                                               _I64, _I64, _I64, _P, _I64, _P, _I, _I64, _I64,
                                               _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64,
                                               _I64, _I64, _I, _I64, _I64, _I64, _I64, _I, _I, _I,
                                               _I, _I64, _I64, _I64, _P]),
    "marlin_dequantize": (_I, [_P, _I64, _P, _I, _I64, _I64, _P, _I, _I64, _P, _I64, _I64, _I64,
                               _I64, _I, _P, _P]),
    "marlin_moe_sum": (_I, [_P, _I, _I64, _I64, _I64, _P, _P]),
    "marlin_silu_and_mul": (_I, [_P, _I, _I64, _I64, _P, _P]),
    "marlin_topk_softmax": (_I, [_P, _P, _I, _P, _I64, _P, _I, _I64, _I64, _I, _P, _I64, _P]),
    "marlin_topk_sigmoid": (_I, [_P, _P, _I, _P, _I64, _P, _I, _I64, _I64, _I, _P, _I64, _P]),
    "marlin_grouped_topk": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _I, ctypes.c_double, _P,
                                 _I, _I64, _I64, _P, _P, _P]),
}

_lib = None


class MarlinError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(msg)
        self.status = status


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing; build it with `python -m marlin_v100_amd.build`")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _numel(t):
    return 0 if t is None else t.numel()


def _dt(t, default=F16):
    return default if t is None else _DT[t.dtype]


def _stream(dev=None):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _check(status: int):
    if status != STATUS_OK:
        raise MarlinError(status, load().marlin_get_last_error().decode())


def gptq_marlin_repack(b_q_weight, perm, size_k, size_n, num_bits, is_a_8bit=False, out=None):
    pack = 32 // num_bits
    if out is None:
        out = torch.empty((size_k // 16, size_n * 16 // pack), dtype=torch.int32,
                          device=b_q_weight.device)
    perm = perm if (perm is not None and perm.numel()) else None
    _check(load().marlin_gptq_marlin_repack(_ptr(b_q_weight), b_q_weight.numel(), _ptr(perm),
                                            _numel(perm), size_k, size_n, num_bits,
                                            int(is_a_8bit), _ptr(out), out.numel(), _stream()))
    return out


def awq_marlin_repack(b_q_weight, size_k, size_n, num_bits, is_a_8bit=False, out=None):
    pack = 32 // num_bits
    if out is None:
        out = torch.empty((size_k // 16, size_n * 16 // pack), dtype=torch.int32,
                          device=b_q_weight.device)
    _check(load().marlin_awq_marlin_repack(_ptr(b_q_weight), b_q_weight.numel(), size_k, size_n,
                                           num_bits, int(is_a_8bit), _ptr(out), out.numel(),
                                           _stream()))
    return out


def marlin_int4_fp8_preprocess(qweight, qzeros=None, out=None):
    """qzeros None: GPTQ-style codes (any shape); else AWQ [size_k, size_n/8] with zero points
    [size_k/group_size, size_n/8].  out may be qweight (in place)."""
    if out is None:
        out = torch.empty_like(qweight)
    rows = qweight.shape[0] if qweight.dim() else 1
    cols = qweight.numel() // rows if rows else 0
    zr, zc = (qzeros.shape[0], qzeros.shape[1]) if qzeros is not None else (0, 0)
    _check(load().marlin_int4_fp8_preprocess(_ptr(qweight), rows, cols, _ptr(qzeros), zr, zc,
                                             _ptr(out), _stream()))
    return out


def marlin_gemm(a, b_q_weight, b_scales, b_type_id, size_m, size_n, size_k, *, c=None,
                b_bias=None, global_scale=None, b_zeros=None, is_zp_float=False, a_scales=None,
                g_idx=None, perm=None, is_k_full=True):
    if c is None:
        c = torch.empty((size_m, size_n), dtype=a.dtype, device=a.device)
    zeros = b_zeros if (b_zeros is not None and b_zeros.numel()) else None
    g_idx = g_idx if (g_idx is not None and g_idx.numel()) else None
    perm = perm if (perm is not None and perm.numel()) else None
    _check(load().marlin_gemm(
        _ptr(a), _dt(a), a.stride(0), _ptr(c), _ptr(b_q_weight), b_q_weight.numel(),
        _ptr(b_bias), _numel(b_bias), _ptr(b_scales), _dt(b_scales), b_scales.numel(),
        b_scales.shape[0], _numel(a_scales), _ptr(global_scale), _numel(global_scale),
        _ptr(zeros), _dt(zeros), _numel(zeros), _ptr(g_idx), _numel(g_idx), _ptr(perm),
        _numel(perm), None, 0, b_type_id, size_m, size_n, size_k, int(is_k_full), 0, 0,
        int(is_zp_float), _stream()))
    return c


def marlin_gemm_no_alloc(a, b_q_weight, b_scales, b_type_id, size_m, size_n, size_k, *, c=None,
                         b_bias=None, global_scale=None, b_zeros=None, is_zp_float=False):
    """marlin_gemm through the entry point that allocates no device memory (the split-K
    scratch is the library's static per-GPU array)."""
    if c is None:
        c = torch.empty((size_m, size_n), dtype=a.dtype, device=a.device)
    zeros = b_zeros if (b_zeros is not None and b_zeros.numel()) else None
    _check(load().marlin_gemm_no_alloc(
        _ptr(a), _dt(a), a.stride(0), _ptr(c), _ptr(b_q_weight), b_q_weight.numel(),
        _ptr(b_bias), _numel(b_bias), _ptr(b_scales), _dt(b_scales), b_scales.numel(),
        b_scales.shape[0], 0, _ptr(global_scale), _numel(global_scale), _ptr(zeros), _dt(zeros),
        _numel(zeros), 0, 0, b_type_id, size_m, size_n, size_k, int(is_zp_float), _stream()))
    return c


def moe_align_block_size(topk_ids, num_experts, block_size, sorted_token_ids, expert_ids,
                         num_tokens_post_pad, expert_map=None):
    _check(load().marlin_moe_align_block_size(
        _ptr(topk_ids), _dt(topk_ids), topk_ids.numel(), num_experts, block_size,
        _ptr(sorted_token_ids), sorted_token_ids.numel(), _ptr(expert_ids), expert_ids.numel(),
        _ptr(num_tokens_post_pad), _ptr(expert_map), _numel(expert_map), _stream()))


def moe_wna16_marlin_gemm(a, b_q_weight, b_scales, sorted_token_ids, expert_ids,
                          num_tokens_past_padded, topk_weights, moe_block_size, top_k,
                          mul_topk_weights, b_type_id, size_m, size_n, size_k, *, c=None,
                          b_bias=None, global_scale=None, b_zeros=None, is_zp_float=False,
                          silu_gated=False):
    """silu_gated: the fused stage-1 entry (c gets silu(h[:, :N/2]) * h[:, N/2:]); raises
    MarlinError with STATUS_NOT_SUPPORTED when the plan cannot fuse it."""
    out_n = size_n // 2 if silu_gated else size_n
    if c is None:
        c = torch.empty((size_m * top_k, out_n), dtype=a.dtype, device=a.device)
    zeros = b_zeros if (b_zeros is not None and b_zeros.numel()) else None
    fn = load().marlin_moe_wna16_marlin_gemm_silu if silu_gated else load().marlin_moe_wna16_marlin_gemm
    _check(fn(
        _ptr(a), _dt(a), _ptr(c), _ptr(b_q_weight), b_q_weight.numel(), b_q_weight.shape[0],
        _ptr(b_bias), _numel(b_bias), _ptr(b_scales), _dt(b_scales), b_scales.numel(),
        b_scales.shape[1], 0, _ptr(global_scale), _numel(global_scale), _ptr(zeros), _dt(zeros),
        _numel(zeros), 0, 0, None, 0, _ptr(sorted_token_ids), sorted_token_ids.numel(),
        _ptr(expert_ids), expert_ids.numel(), _ptr(num_tokens_past_padded), _ptr(topk_weights),
        _numel(topk_weights), moe_block_size, top_k, int(mul_topk_weights), b_type_id, size_m,
        size_n, size_k, 1, 0, 0, int(is_zp_float), -1, -1, -1, _stream()))
    return c


def dequantize(b_q_weight, b_scales, b_type_id, size_k, size_n, out_dtype, *, b_zeros=None,
               global_scale=None):
    out = torch.empty((size_k, size_n), dtype=out_dtype, device=b_q_weight.device)
    zeros = b_zeros if (b_zeros is not None and b_zeros.numel()) else None
    _check(load().marlin_dequantize(
        _ptr(b_q_weight), b_q_weight.numel(), _ptr(b_scales), _dt(b_scales), b_scales.numel(),
        b_scales.shape[0], _ptr(zeros), _dt(zeros), _numel(zeros), _ptr(global_scale),
        _numel(global_scale), b_type_id, size_k, size_n, _DT[out_dtype], _ptr(out), _stream()))
    return out


def moe_sum(inp, out):
    _check(load().marlin_moe_sum(_ptr(inp), _dt(inp), inp.shape[0], inp.shape[1], inp.shape[2],
                                 _ptr(out), _stream()))
    return out


def silu_and_mul(out, x):
    """out[r, :] = silu(x[r, :d]) * x[r, d:] for contiguous x [rows, 2d], out [rows, d]."""
    d = x.shape[-1] // 2
    rows = x.numel() // max(2 * d, 1)
    _check(load().marlin_silu_and_mul(_ptr(x), _dt(x), rows, d, _ptr(out), _stream()))
    return out


def topk_gating(gating, topk, renormalize=False, bias=None, scoring="softmax",
                ids_dtype=torch.int32):
    """Router top-k over gating [T, E]: returns (weights f32, ids, token_expert_indices)."""
    t, e = gating.shape
    dev = gating.device
    w = torch.empty((t, topk), dtype=torch.float32, device=dev)
    ids = torch.empty((t, topk), dtype=ids_dtype, device=dev)
    tei = torch.empty((t, topk), dtype=torch.int32, device=dev)
    fn = load().marlin_topk_softmax if scoring == "softmax" else load().marlin_topk_sigmoid
    _check(fn(_ptr(w), _ptr(ids), _DT[ids_dtype], _ptr(tei), topk, _ptr(gating), _dt(gating), t,
              e, int(renormalize), _ptr(bias), _numel(bias), _stream()))
    return w, ids, tei


def grouped_topk(scores, n_group, topk_group, topk, renormalize, routed_scaling_factor, bias,
                 scoring_func=0):
    """Grouped router over scores [T, E]: returns (values f32 [T, topk], ids i32 [T, topk])."""
    t, e = scores.shape
    vals = torch.empty((t, topk), dtype=torch.float32, device=scores.device)
    ids = torch.empty((t, topk), dtype=torch.int32, device=scores.device)
    _check(load().marlin_grouped_topk(_ptr(scores), _dt(scores), t, e, n_group, topk_group, topk,
                                      int(renormalize), float(routed_scaling_factor), _ptr(bias),
                                      _dt(bias), _numel(bias), scoring_func, _ptr(vals),
                                      _ptr(ids), _stream()))
    return vals, ids
