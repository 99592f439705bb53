"""CPU restatement of the reference Marlin semantics (torch on CPU, numpy for integer work).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; never by the product package.

All `file:line` citations point into the reference tree zhinianqin/marlin_v100.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

# ---------------------------------------------------------------------------------------
# Scalar types (vllm/scalar_type.py:25-43, 83-90; tests/helpers.py:14-57)
# ---------------------------------------------------------------------------------------


@dataclass(frozen=True)
class ScalarType:
    exponent: int
    mantissa: int
    signed: bool
    bias: int = 0
    finite_values_only: bool = False
    nan_repr: int = 1

    @property
    def size_bits(self) -> int:
        return self.exponent + self.mantissa + int(self.signed)

    @property
    def id(self) -> int:
        # fields packed LSB first: exponent:8 mantissa:8 signed:1 bias:32 finite:1 nan:8
        val, off = 0, 0
        for member, width in ((self.exponent, 8), (self.mantissa, 8), (self.signed, 1),
                              (self.bias, 32), (self.finite_values_only, 1),
                              (self.nan_repr, 8)):
            val |= (int(member) & ((1 << width) - 1)) << off
            off += width
        return val


class scalar_types:
    uint4 = ScalarType(0, 4, False, 0)
    uint4b8 = ScalarType(0, 4, False, 8)
    uint8 = ScalarType(0, 8, False, 0)
    uint8b128 = ScalarType(0, 8, False, 128)
    float4_e2m1f = ScalarType(2, 1, True, 0, True, 0)
    float8_e4m3fn = ScalarType(4, 3, True, 0, True, 2)
    float8_e8m0fnu = ScalarType(8, 0, False, 0, True, 2)


# ---------------------------------------------------------------------------------------
# Packing conventions
# ---------------------------------------------------------------------------------------

def gptq_pack(q: torch.Tensor, num_bits: int) -> torch.Tensor:
    """[K, N] ints -> [K/pack, N] int32, value k = pack*r + i in bits [i*b, (i+1)*b).
    tests/helpers.py:401-426 (pack_rows)."""
    k, n = q.shape
    pack = 32 // num_bits
    assert k % pack == 0
    qn = q.to(torch.int64).reshape(k // pack, pack, n)
    out = torch.zeros((k // pack, n), dtype=torch.int64)
    for i in range(pack):
        out |= (qn[:, i, :] & ((1 << num_bits) - 1)) << (num_bits * i)
    return _to_i32(out)


def _to_i32(x: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(x.numpy().astype(np.uint32).view(np.int32))


def awq_pack(q: torch.Tensor, num_bits: int) -> torch.Tensor:
    """[K, N] ints -> [K, N/pack] int32 with the AWQ column interleave
    {0,2,4,6,1,3,5,7} (4-bit) / {0,2,1,3} (8-bit).  tests/helpers.py:548-562, 429-446."""
    k, n = q.shape
    pack = 32 // num_bits
    order = [0, 2, 4, 6, 1, 3, 5, 7] if num_bits == 4 else [0, 2, 1, 3]
    qi = q.to(torch.int64).reshape(-1, pack)[:, order].reshape(k, n)
    out = torch.zeros((k, n // pack), dtype=torch.int64)
    for i in range(pack):
        out |= (qi[:, i::pack] & ((1 << num_bits) - 1)) << (num_bits * i)
    return _to_i32(out)


def fp4_to_gptq_words(q_nibbles_kn: torch.Tensor) -> torch.Tensor:
    """FP4 codes [K, N] -> the GPTQ-style [K/8, N] int32 the FP4 layer path feeds to
    gptq_marlin_repack: checkpoint bytes [N, K/2] (low nibble = even k) viewed as int32
    and transposed (marlin_utils_fp4.py:229)."""
    k, n = q_nibbles_kn.shape
    qn = q_nibbles_kn.to(torch.int64).T.contiguous()  # [N, K]
    bytes_nk = (qn[:, 0::2] | (qn[:, 1::2] << 4)).to(torch.uint8)  # [N, K/2]
    words = bytes_nk.contiguous().view(torch.int32)  # [N, K/8]
    return words.T.contiguous()


def unpack_gptq(words: torch.Tensor, num_bits: int) -> torch.Tensor:
    kp, n = words.shape
    pack = 32 // num_bits
    w = words.to(torch.int64) & 0xFFFFFFFF
    out = torch.empty((kp * pack, n), dtype=torch.int64)
    for i in range(pack):
        out[i::pack] = (w >> (num_bits * i)) & ((1 << num_bits) - 1)
    return out.to(torch.int32)


def a8_layout_index(size_k: int, size_n: int, num_bits: int):
    """Source coordinates of every code slot of the reference's 8-bit-activation repack output
    (is_a_8bit; gptq_marlin_repack.cu:225-335, awq_marlin_repack.cu:165-270): arrays
    (k, n) of shape [words, pack], slot i of output word w holding code (k[w, i], n[w, i]).
    32 x 32 (k x n) tiles, k tiles outer, 32*32/pack words each; word group (thread th,
    n8 slice s) covers column 16*(s//2) + 8*(s%2) + th//4 and rows 4*(th%4) + {0..3} and the
    same rows + 16 -- for 4-bit one word th*4 + s (pack_idx {0,4,1,5,2,6,3,7}: nibble i =
    row + i//2 + 16*(i%2)), for 8-bit two words th*8 + 2*s + h (byte i = row + 16*h + i)."""
    pack = 32 // num_bits
    assert size_k % 32 == 0 and size_n % 32 == 0
    tile_words = 32 * 32 // pack
    words = size_k * size_n // pack
    w = np.arange(words, dtype=np.int64)
    tile, r = w // tile_words, w % tile_words
    n_tiles = size_n // 32
    kt, nt = tile // n_tiles, tile % n_tiles
    if num_bits == 4:
        th, s, h = r // 4, r % 4, np.zeros_like(r)
    else:
        th, s, h = r // 8, (r // 2) % 4, r % 2
    n = nt * 32 + 16 * (s // 2) + 8 * (s % 2) + th // 4
    k0 = kt * 32 + 4 * (th % 4)
    i = np.arange(pack, dtype=np.int64)[None, :]
    if num_bits == 4:
        k = k0[:, None] + i // 2 + 16 * (i % 2)
    else:
        k = k0[:, None] + 16 * h[:, None] + i
    return k, np.broadcast_to(n[:, None], k.shape)


def a8_repack(q: np.ndarray, num_bits: int) -> np.ndarray:
    """Logical codes q [K, N] -> the 8-bit-activation repack output as int32
    [K/16, N*16/pack] (a8_layout_index)."""
    size_k, size_n = q.shape
    pack = 32 // num_bits
    k, n = a8_layout_index(size_k, size_n, num_bits)
    codes = q.astype(np.uint64)[k, n] & ((1 << num_bits) - 1)
    shifts = (np.arange(pack, dtype=np.uint64) * num_bits)[None, :]
    words = (codes << shifts).sum(axis=1).astype(np.uint32)
    return words.view(np.int32).reshape(size_k // 16, size_n * 16 // pack)


def int4_fp8_preprocess(words: np.ndarray, zeros: np.ndarray | None = None) -> np.ndarray:
    """marlin_int4_fp8_preprocess.cu:8-56: every 4-bit code v becomes v - z if v >= z else
    15 - v, with z = 8 (no zero points) or the code's AWQ zero point (same word column and
    nibble, zero-point row k // group_size for weights [K, N/8], zero points [K/gs, N/8])."""
    w = words.astype(np.int64) & 0xFFFFFFFF
    if zeros is None:
        z = np.full_like(w, 0x88888888)
    else:
        gs = words.shape[0] // zeros.shape[0]
        z = np.repeat(zeros.astype(np.int64) & 0xFFFFFFFF, gs, axis=0)
    out = np.zeros_like(w)
    for i in range(8):
        v = (w >> (4 * i)) & 15
        zz = (z >> (4 * i)) & 15
        out |= np.where(v >= zz, v - zz, 15 - v) << (4 * i)
    return out.astype(np.uint32).view(np.int32).reshape(words.shape)


# ---------------------------------------------------------------------------------------
# e2m1 / e8m0 / e4m3 helpers
# ---------------------------------------------------------------------------------------
# e2m1 code -> value (tests/helpers.py:742-764)
FP4_VALUES = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                           -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=torch.float32)


def quantize_to_fp4_e2m1(values: torch.Tensor) -> torch.Tensor:
    """Nearest e2m1 code, first index on ties (tests/helpers.py:767-770)."""
    d = (values.to(torch.float32).unsqueeze(-1) - FP4_VALUES).abs()
    return d.argmin(dim=-1).to(torch.int32)


# ---------------------------------------------------------------------------------------
# Quantizers (the build's own seeded generators follow the reference helpers' formulas)
# ---------------------------------------------------------------------------------------

def _groups(k: int, gs: int) -> int:
    return 1 if gs == -1 else k // gs


def quantize_with_bias(w: torch.Tensor, gs: int, bias: int, dtype: torch.dtype):
    """Symmetric RTN to uint with bias (u4b8: bias 8, u8b128: bias 128).
    s = dtype(max|w| / (bias-1)), q = clamp(round(w/s), -bias, bias-1) + bias.
    tests/helpers.py:641-658."""
    k, n = w.shape
    g = _groups(k, gs)
    r = w.to(torch.float32).reshape(g, k // g, n)
    s = (r.abs().amax(dim=1) / float(bias - 1)).clamp_min(1e-6).to(dtype)
    q = torch.round(r / s.to(torch.float32).unsqueeze(1)).clamp(-bias, bias - 1) + bias
    return q.to(torch.int32).reshape(k, n), s


def quantize_with_zero_point(w: torch.Tensor, gs: int, bits: int, dtype: torch.dtype):
    """Asymmetric RTN: s = (max-min)/(2^b-1), z = clamp(round(-min/s)), q = clamp(round(w/s+z)).
    Returns q, s (dtype), z (int), zp_f = dtype(z*s) (the float zero point the kernel takes,
    tests/helpers.py:1249, marlin_utils.py:451).  tests/helpers.py:661-698."""
    k, n = w.shape
    g = _groups(k, gs)
    qmax = (1 << bits) - 1
    r = w.to(torch.float32).reshape(g, k // g, n)
    mins, maxs = r.amin(dim=1), r.amax(dim=1)
    s32 = ((maxs - mins) / float(qmax)).clamp_min(1e-6)
    z = torch.round(-mins / s32).clamp(0, qmax).to(torch.int32)
    q = torch.round(r / s32.unsqueeze(1) + z.unsqueeze(1)).clamp(0, qmax).to(torch.int32)
    s = s32.to(dtype)
    zp_f = (z.to(torch.float32) * s.to(torch.float32)).to(dtype)
    return q.reshape(k, n), s, z, zp_f


def quantize_mxfp4(w: torch.Tensor, gs: int = 32):
    """MXFP4: e8m0 scale 2^ceil(log2(max|w|/6)) per 32 k, e2m1 codes of w/scale.
    tests/helpers.py:857-887."""
    assert gs == 32
    k, n = w.shape
    r = w.to(torch.float32).reshape(k // gs, gs, n)
    max_abs = r.abs().amax(dim=1)
    inp = torch.where(max_abs > 0, (max_abs / 6.0).clamp_min(2.0 ** -127), torch.ones_like(max_abs))
    e = torch.ceil(torch.log2(inp)).clamp(-127, 127)
    scales = torch.pow(torch.full_like(e, 2.0), e).to(torch.float8_e8m0fnu)
    eff = scales.to(torch.float32)
    q = quantize_to_fp4_e2m1(r / eff.unsqueeze(1).clamp_min(1e-12)).reshape(k, n)
    return q, scales


def quantize_nvfp4(w: torch.Tensor, gs: int = 16):
    """NVFP4: per-16 scale max|w|/6 stored as e4m3 relative to global = max(scale)/448.
    tests/helpers.py:831-854."""
    assert gs == 16
    k, n = w.shape
    r = w.to(torch.float32).reshape(k // gs, gs, n)
    sc = (r.abs().amax(dim=1) / 6.0).clamp_min(1e-6)
    glob = (sc.max() / 448.0).to(torch.float32).reshape(1)
    fp8 = (sc / glob).to(torch.float8_e4m3fn)
    eff = fp8.to(torch.float32) * glob
    q = quantize_to_fp4_e2m1(r / eff.unsqueeze(1).clamp_min(1e-12)).reshape(k, n)
    return q, fp8, glob


def quantize_fp8(w: torch.Tensor, gs: int, dtype: torch.dtype):
    """fp8-e4m3 weights with scale max|w|/448 per group; the kernel scale is
    dtype(scale * 256) (exponent-bias fold).  tests/helpers.py:890-911, 701-703."""
    k, n = w.shape
    g = _groups(k, gs)
    r = w.to(torch.float32).reshape(g, k // g, n)
    s = (r.abs().amax(dim=1) / 448.0).clamp_min(1e-6)
    fp8 = (r / s.unsqueeze(1)).to(torch.float8_e4m3fn).reshape(k, n)
    return fp8, (s * 256.0).to(dtype)


# ---------------------------------------------------------------------------------------
# Metadata preprocessing (marlin_utils*.py)
# ---------------------------------------------------------------------------------------
_SCALE_PERM_SINGLE = [2 * i + j for i in range(4) for j in (0, 1, 8, 9, 16, 17, 24, 25)]


def marlin_permute_bias(bias: torch.Tensor) -> torch.Tensor:
    """marlin_utils.py:279-286, 310-314."""
    shape = bias.shape
    return bias.reshape(-1, 32)[:, _SCALE_PERM_SINGLE].reshape(shape).contiguous()


def nvfp4_compute_scale_factor(scales: torch.Tensor, a_dtype: torch.dtype) -> float:
    """marlin_utils_fp4.py:30-50."""
    if a_dtype == torch.float16:
        return 1.0
    ws = scales.float() * (2 ** 7)
    nz = ws > 0
    if nz.any():
        mn = ws[nz].min()
        if mn < 2:
            return float((2 / mn).log2().ceil().exp2().item())
    return 1.0


def nvfp4_marlin_process_scales(scales_e4m3: torch.Tensor, a_dtype: torch.dtype,
                                scale_factor: float | None = None):
    """e4m3 [G, N] -> S0E5M3 bytes [G, N] with a [0,2,1,3] shuffle per 4 columns.
    marlin_utils_fp4.py:53-110."""
    s = scales_e4m3.to(torch.float16)
    s = s.view(-1, 4)[:, [0, 2, 1, 3]].reshape(s.shape)
    if scale_factor is None:
        scale_factor = nvfp4_compute_scale_factor(s, a_dtype)
    if scale_factor > 1.0:
        s = (s.float() * scale_factor).to(torch.float16)
    bits = (s * (2 ** 7)).view(torch.int16) << 1
    out = bits.view(torch.float8_e4m3fn)[:, 1::2].contiguous()
    return out, scale_factor


def nvfp4_exponent_bias(a_dtype: torch.dtype) -> int:
    """2^(target_exp-1) - 2^(fp4_exp-1): 14 for fp16, 126 for bf16 (marlin_utils_fp4.py:132-144)."""
    target = 5 if a_dtype == torch.float16 else 8
    return 2 ** (target - 1) - 2 ** (2 - 1)


def nvfp4_marlin_process_global_scale(glob: torch.Tensor, a_dtype: torch.dtype) -> torch.Tensor:
    """marlin_utils_fp4.py:132-144."""
    return glob * (2.0 ** (nvfp4_exponent_bias(a_dtype) - 7))


def decode_s0e5m3(processed: torch.Tensor) -> torch.Tensor:
    """S0E5M3 bytes -> fp32 scale*2^7*sf in logical column order
    (tests/helpers.py:825-828)."""
    bits = processed.view(torch.uint8).to(torch.int16) << 7
    dec = bits.contiguous().view(torch.float16).to(torch.float32)
    return dec.view(-1, 4)[:, [0, 2, 1, 3]].reshape(processed.shape)


# ---------------------------------------------------------------------------------------
# Dequantization (logical q + metadata -> [K, N] in dtype), one rounding per weight
# ---------------------------------------------------------------------------------------

def _expand(meta: torch.Tensor, k: int) -> torch.Tensor:
    g = meta.shape[0]
    return meta.repeat_interleave(k // g, dim=0)


def dequant_int(q: torch.Tensor, scales: torch.Tensor, fmt: str, out_dtype: torch.dtype,
                zp_f: torch.Tensor | None = None) -> torch.Tensor:
    """u4b8/u8b128: dtype((q - bias) * s) (tests/helpers.py:1122-1133);
    u4/u8 + float zp: dtype(q * s - zp_f) (tests/helpers.py:1576-1641)."""
    k = q.shape[0]
    s = _expand(scales.to(torch.float32), k)
    qf = q.to(torch.float32)
    if fmt in ("u4b8", "u8b128"):
        bias = 8.0 if fmt == "u4b8" else 128.0
        return ((qf - bias) * s).to(out_dtype)
    assert zp_f is not None
    return (qf * s - _expand(zp_f.to(torch.float32), k)).to(out_dtype)


def dequant_int_zero(q: torch.Tensor, scales: torch.Tensor, z: torch.Tensor,
                     out_dtype: torch.dtype, g_idx: torch.Tensor | None = None) -> torch.Tensor:
    """Integer zero points (upstream marlin's is_zp_float=False, marlin_utils.py:347-396):
    dtype((q - z) * s), one rounding of the exact value (the reference rejects this mode,
    marlin.cu:336-339).  g_idx: per-row group index instead of row // group_size."""
    k = q.shape[0]
    if g_idx is None:
        s, zz = _expand(scales.to(torch.float32), k), _expand(z.to(torch.float32), k)
    else:
        s, zz = scales.to(torch.float32)[g_idx.long()], z.to(torch.float32)[g_idx.long()]
    return ((q.to(torch.float32) - zz) * s).to(out_dtype)


def dequant_int_g_idx(q: torch.Tensor, scales: torch.Tensor, fmt: str, out_dtype: torch.dtype,
                      g_idx: torch.Tensor, zp_f: torch.Tensor | None = None) -> torch.Tensor:
    """dequant_int with act-order groups: row k uses scale row g_idx[k]
    (upstream gptq act-order; tests/helpers.py:1122-1133 semantics per row)."""
    gi = g_idx.long()
    s = scales.to(torch.float32)[gi]
    qf = q.to(torch.float32)
    if fmt in ("u4b8", "u8b128"):
        bias = 8.0 if fmt == "u4b8" else 128.0
        return ((qf - bias) * s).to(out_dtype)
    return (qf * s - zp_f.to(torch.float32)[gi]).to(out_dtype)


def act_order_groups(k: int, gs: int, gen: torch.Generator):
    """A GPTQ act-order grouping: a random column order `perm` (GPTQ's descending-activation
    order) and g_idx[perm[j]] = j // gs, so each group holds gs rows and argsort(g_idx)
    returns those groups contiguously (marlin_utils.py:274-276)."""
    perm = torch.randperm(k, generator=gen)
    g_idx = torch.empty(k, dtype=torch.int32)
    g_idx[perm] = (torch.arange(k) // gs).to(torch.int32)
    return g_idx


def quantize_g_idx(w: torch.Tensor, g_idx: torch.Tensor, num_groups: int, fmt: str,
                   dtype: torch.dtype):
    """RTN with act-order groups: the group of row k is g_idx[k].  Returns (q [K, N] codes,
    s [G, N], z [G, N] int or None, zp_f [G, N] or None) with the formulas of
    quantize_with_bias / quantize_with_zero_point applied per group's row set."""
    k, n = w.shape
    bits = 4 if fmt in ("u4b8", "u4") else 8
    q = torch.empty((k, n), dtype=torch.int32)
    ss, zs, zfs = [], [], []
    for g in range(num_groups):
        rows = (g_idx == g).nonzero().flatten()
        if fmt in ("u4b8", "u8b128"):
            qg, sg = quantize_with_bias(w[rows], -1, 8 if fmt == "u4b8" else 128, dtype)
            zg = zfg = None
        else:
            qg, sg, zg, zfg = quantize_with_zero_point(w[rows], -1, bits, dtype)
        q[rows] = qg
        ss.append(sg)
        zs.append(zg)
        zfs.append(zfg)
    s = torch.cat(ss)
    if fmt in ("u4b8", "u8b128"):
        return q, s, None, None
    return q, s, torch.cat(zs), torch.cat(zfs)


def pack_cols(z: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes [G, N] packed along N, 32/bits per int32, column n in bits [bits*(n % pack), ...)
    (quant_utils.py:66-78)."""
    g, n = z.shape
    pack = 32 // bits
    zz = z.to(torch.int64).reshape(g, n // pack, pack)
    out = torch.zeros((g, n // pack), dtype=torch.int64)
    for i in range(pack):
        out |= zz[:, :, i] << (bits * i)
    return _to_i32(out)


def dequant_mxfp4(q: torch.Tensor, scales_e8m0: torch.Tensor, out_dtype: torch.dtype):
    """dtype(e2m1 * 2^(e-127)) (tests/helpers.py:1164-1184)."""
    k = q.shape[0]
    return (FP4_VALUES[q.long()] * _expand(scales_e8m0.to(torch.float32), k)).to(out_dtype)


def dequant_nvfp4(q: torch.Tensor, processed_scales: torch.Tensor, processed_global: torch.Tensor,
                  out_dtype: torch.dtype) -> torch.Tensor:
    """dtype((e2m1 * 2^-bias * decode(S0E5M3)) * global'), products in fp32, bias = 14
    (fp16) or 126 (bf16).  tests/helpers.py:1135-1161 (written there for fp16)."""
    k = q.shape[0]
    bias = nvfp4_exponent_bias(out_dtype)
    vals = FP4_VALUES[q.long()] * (2.0 ** -bias)
    dec = _expand(decode_s0e5m3(processed_scales), k)
    return (vals * dec * processed_global.reshape(-1)[0].to(torch.float32)).to(out_dtype)


def dequant_fp8(fp8_w: torch.Tensor, scales_x256: torch.Tensor, out_dtype: torch.dtype):
    """dtype(fp8 * (s/256)) (tests/helpers.py:1117-1121)."""
    k = fp8_w.shape[0]
    return (fp8_w.to(torch.float32) * (_expand(scales_x256.to(torch.float32), k) / 256.0)).to(out_dtype)


# ---------------------------------------------------------------------------------------
# GEMM reference (tests/helpers.py:1749-1760): dequantize, then fp32 matmul
# ---------------------------------------------------------------------------------------

def gemm_ref(a: torch.Tensor, w_deq: torch.Tensor, bias: torch.Tensor | None = None,
             alpha: float = 1.0) -> torch.Tensor:
    out = torch.matmul(a.to(torch.float32), w_deq.to(torch.float32)) * alpha
    if bias is not None:
        out = out + bias.to(torch.float32)
    return out


def moe_sum(x: torch.Tensor) -> torch.Tensor:
    """out[t, h] = sum_k x[t, k, h] for x [T, topk, H] in fp16/bf16, as the reference computes
    it (csrc/moe/moe_align_sum_kernels.cu:350-363, 597-639): top-k 2..4 run its kernel, which
    adds in the element type (one rounding per addition, k in order); every other top-k
    falls through to at::sum_out (fp32 accumulation in k order, one rounding)."""
    topk = x.shape[1]
    step = 2 <= topk <= 4
    s = torch.zeros(x[:, 0].shape, dtype=torch.float32)
    for k in range(topk):
        s = s + x[:, k].float()
        if step:
            s = s.to(x.dtype).float()
    return s.to(x.dtype)


# ---------------------------------------------------------------------------------------
# moe_align_block_size (tests/test_marlin_moe.py:194-213 order; tail rules from
# csrc/moe/moe_align_sum_kernels.cu:101-108, 126-133, 168-180)
# ---------------------------------------------------------------------------------------

def moe_align_block_size(topk_ids: np.ndarray, num_experts: int, block_size: int,
                         sorted_numel: int | None = None, expert_ids_numel: int | None = None,
                         expert_map: np.ndarray | None = None):
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    numel = flat.size
    if sorted_numel is None:
        sorted_numel = numel + num_experts * (block_size - 1)
    if expert_ids_numel is None:
        expert_ids_numel = sorted_numel // block_size + 1
    mapped = np.full(numel, -1, dtype=np.int64)
    ok = (flat >= 0) & (flat < num_experts)
    mapped[ok] = flat[ok]
    if expert_map is not None:
        em = np.asarray(expert_map).astype(np.int64)
        mapped[ok] = em[flat[ok]]
        mapped[(mapped < 0) | (mapped >= num_experts)] = -1
    sorted_ids = np.full(sorted_numel, numel, dtype=np.int32)
    expert_ids = np.full(expert_ids_numel, -1, dtype=np.int32)
    pos = 0
    for e in range(num_experts):
        idx = np.nonzero(mapped == e)[0]
        padded = (idx.size + block_size - 1) // block_size * block_size
        if padded == 0:
            continue
        sorted_ids[pos:pos + idx.size] = idx
        expert_ids[pos // block_size:(pos + padded) // block_size] = e
        pos += padded
    return sorted_ids, expert_ids, np.array([pos], dtype=np.int32)


# ---------------------------------------------------------------------------------------
# MoE layer reference (tests/helpers.py:2039-2060 math, vectorized per expert;
# orchestration per fused_marlin_moe.py:50-382: gate = first half, silu(gate) * up)
# ---------------------------------------------------------------------------------------

def moe_layer_ref(x: torch.Tensor, w13_deq: torch.Tensor, w2_deq: torch.Tensor,
                  topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
    """x [T, H]; w13_deq [E, H, 2I]; w2_deq [E, I, H]; returns fp32 [T, H]."""
    t, h = x.shape
    topk = topk_ids.shape[1]
    inter = w2_deq.shape[1]
    out = torch.zeros((t, h), dtype=torch.float32)
    xf = x.to(torch.float32)
    flat_ids = topk_ids.reshape(-1).long()
    tok = torch.arange(t).repeat_interleave(topk)
    wts = topk_weights.reshape(-1).to(torch.float32)
    for e in torch.unique(flat_ids).tolist():
        sel = (flat_ids == e).nonzero().reshape(-1)
        rows = tok[sel]
        g = xf[rows] @ w13_deq[e].to(torch.float32)
        act = torch.nn.functional.silu(g[:, :inter]) * g[:, inter:]
        y = act @ w2_deq[e].to(torch.float32)
        out.index_add_(0, rows, y * wts[sel].unsqueeze(1))
    return out


def route_topk(logits: torch.Tensor, topk: int):
    """softmax (fp32) -> top-k -> renormalise (the BASELINE router)."""
    p = torch.softmax(logits.to(torch.float32), dim=-1)
    w, ids = torch.topk(p, topk, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return w.contiguous(), ids.to(torch.int32).contiguous()


# ---------------------------------------------------------------------------------------
# MoE router: topk_softmax / topk_sigmoid (reference test oracle tests/test_marlin_moe.py:111-133;
# kernel rules csrc/moe/topk_softmax_kernels.cu: softmax :75-133, sigmoid :135-153, selection by
# score + bias with ties to the lower expert index :446-460, :488, :508, unbiased output
# weights :223-225, renormalization by the chosen sum with a zero sum dividing by 1 :551-560,
# token_expert_indices = j * T + t :226, :527)
# ---------------------------------------------------------------------------------------

def topk_gating(gating: np.ndarray, topk: int, renormalize: bool = False,
                bias: np.ndarray | None = None, scoring: str = "softmax"):
    """gating [T, E] (any float dtype); returns (weights f32 [T, k], ids i32 [T, k],
    token_expert_indices i32 [T, k]).  Scores are computed in float32."""
    x = np.asarray(gating, dtype=np.float32)
    t, e = x.shape
    if scoring == "softmax":
        ex = np.exp(x - x.max(axis=1, keepdims=True), dtype=np.float32)
        scores = (ex / ex.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    elif scoring == "sigmoid":
        scores = (np.float32(1.0) / (np.float32(1.0) + np.exp(-x, dtype=np.float32))).astype(
            np.float32)
    else:
        raise ValueError(scoring)
    choice = scores if bias is None else (scores + np.asarray(bias, np.float32)[None, :])
    # descending choice, ties to the lower index: lexsort's last key is the primary one
    cols = np.arange(e)
    ids = np.empty((t, topk), dtype=np.int32)
    for r in range(t):
        order = np.lexsort((cols, -choice[r].astype(np.float64)))
        ids[r] = order[:topk]
    w = np.take_along_axis(scores, ids.astype(np.int64), axis=1).astype(np.float32)
    if renormalize:
        s = w.sum(axis=1, keepdims=True, dtype=np.float32)
        w = (w / np.where(s > 0, s, np.float32(1.0))).astype(np.float32)
    tei = (np.arange(topk, dtype=np.int64)[None, :] * t + np.arange(t)[:, None]).astype(np.int32)
    return w, ids, tei


# ---------------------------------------------------------------------------------------
# MoE grouped router: grouped_topk (reference test oracle tests/test_marlin_moe.py:136-191;
# kernel rules csrc/moe/grouped_topk_kernels.cu: group score = sum of the two largest
# score + bias :469-512, kept groups :576-585, non-finite inputs never compete :623-628,
# weights = unbiased score * routed_scaling_factor / (1e-20 + sum) :639-656, fallback to
# experts 0..k-1 with weight 1/k when the last kept group scores -inf :587-600)
# ---------------------------------------------------------------------------------------

def grouped_topk(scores: np.ndarray, n_group: int, topk_group: int, topk: int,
                 renormalize: bool, routed_scaling_factor: float, bias: np.ndarray,
                 scoring_func: int = 0):
    """scores [T, E]; returns (values f32 [T, topk], ids i32 [T, topk])."""
    x = np.asarray(scores, dtype=np.float32)
    t, e = x.shape
    epg = e // n_group
    if scoring_func == 0:
        unbiased = x
    elif scoring_func == 1:
        unbiased = (np.float32(1.0) / (np.float32(1.0) + np.exp(-x, dtype=np.float32))).astype(
            np.float32)
    else:
        raise ValueError(scoring_func)
    biased = np.where(np.isfinite(x), unbiased + np.asarray(bias, np.float32)[None, :],
                      np.float32(-np.inf)).astype(np.float32)
    values = np.empty((t, topk), dtype=np.float32)
    ids = np.empty((t, topk), dtype=np.int32)
    for r in range(t):
        gsc = []
        for g in range(n_group):
            top = np.sort(biased[r, g * epg:(g + 1) * epg])[::-1][:min(2, epg)]
            gsc.append((float(np.float32(top.sum(dtype=np.float32))), g))
        kept = sorted(gsc, key=lambda it: (-it[0], it[1]))[:topk_group]
        if not kept[-1][0] > -np.inf:
            ids[r] = np.arange(topk)
            values[r] = np.float32(1.0 / topk)
            continue
        cand = [(float(biased[r, ex]), ex) for _, g in kept for ex in range(g * epg, (g + 1) * epg)]
        sel = [ex for _, ex in sorted(cand, key=lambda it: (-it[0], it[1]))[:topk]]
        w = unbiased[r, sel].astype(np.float32)
        scale = np.float32(routed_scaling_factor)
        if renormalize:
            scale = np.float32(scale / (np.float32(1e-20) + w.sum(dtype=np.float32)))
        ids[r] = sel
        values[r] = w * scale
    return values, ids


def max_abs_rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max|out - ref| / max|ref| (the BASELINE tolerance metric)."""
    ref = ref.to(torch.float32)
    den = ref.abs().max().item()
    return (out.to(torch.float32) - ref).abs().max().item() / (den if den > 0 else 1.0)


__all__ = [n for n in dir() if not n.startswith("_")]
