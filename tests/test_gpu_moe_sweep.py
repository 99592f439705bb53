"""Seeded random sweep of moe_wna16_marlin_gemm against the oracle, route by route: formats
with >= 128-deep groups, channelwise scales and fp4, both dtypes, 2-16 experts, top-k 1-4,
1-300 tokens (so both the few-routes decode kernel and the multistage / tiled moe blocks),
every moe block size, K any multiple of 128 up to 1536, size_n any multiple of 64 up to 1024,
with and without router weights and a bias.  Bar: max|out - ref| <= 1e-2 * max|ref|.
As in the reference's MoE epilogue and bias init (moe sm70_marlin_gemm.cuh:3490-3503,
sm70_marlin_bias.cu:56-58), an NVFP4 bias under router weights is multiplied by the global
scale as passed to the op."""
import math
import random

import numpy as np
import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from tests.quant_cases import BITS, make_case

pytestmark = pytest.mark.gpu

TOL = 1e-2
FMTS = ("u4b8", "u4", "u8b128", "u8", "fp8", "mxfp4", "nvfp4")


def _case(i):
    rng = random.Random(7000 + i)
    fmt = FMTS[i % len(FMTS)]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    e = rng.randint(2, 16)
    topk = rng.randint(1, min(4, e))
    t = max(1, int(round(2 ** rng.uniform(0, math.log2(300)))))
    bs = rng.choice([8, 16, 32, 48, 64])
    k = 128 * rng.randint(1, 12)
    n = 64 * rng.randint(1, 16)
    mul = rng.random() < 0.5
    bias = rng.random() < 0.33
    return fmt, dtype, e, topk, t, bs, k, n, mul, bias


CASES = [_case(i) for i in range(70)]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_moe_gemm_random_shapes(i):
    fmt, dtype, E, topk, T, bs, K, N, mul, bias = CASES[i]
    print(f"case moe-sweep {i}: fmt={fmt} dtype={dtype} E={E} topk={topk} T={T} bs={bs} K={K} "
          f"N={N} mul={mul} bias={bias}", flush=True)
    cases = [make_case(fmt, K, N, dtype, seed=800 + 31 * i + j) for j in range(E)]
    words = torch.stack([capi.gptq_marlin_repack(c.gptq_words.cuda(), None, K, N, BITS[fmt])
                         for c in cases])
    scales = torch.stack([c.scales for c in cases]).cuda()
    zeros = torch.stack([c.zeros for c in cases]).cuda() if cases[0].zeros is not None else None
    glob = (torch.cat([c.global_scale for c in cases]).cuda()
            if cases[0].global_scale is not None else None)
    gen = torch.Generator().manual_seed(900 + i)
    x = torch.randn((T, K), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    b = (torch.randn((E, N), generator=gen) * 0.1).to(dtype) if bias else None
    out = capi.moe_wna16_marlin_gemm(
        x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(), tw.cuda(), bs, topk, mul,
        cases[0].type_id, T, N, K, b_zeros=zeros, global_scale=glob,
        is_zp_float=zeros is not None,
        b_bias=torch.stack([O.marlin_permute_bias(b[j]) for j in range(E)]).cuda()
        if bias else None).cpu()
    flat = ids.reshape(-1)
    ref = torch.empty((flat.numel(), N))
    for r in range(flat.numel()):
        v = x[r // topk].float() @ cases[int(flat[r])].deq.float()
        if bias:
            g = float(glob[flat[r]]) if fmt == "nvfp4" and mul else 1.0
            v = v + b[flat[r]].float() * g
        ref[r] = v * tw.reshape(-1)[r] if mul else v
    assert O.max_abs_rel_err(out, ref) <= TOL


def _align_case(i):
    rng = random.Random(7500 + i)
    e = max(1, int(round(2 ** rng.uniform(0, 10))))
    topk = rng.randint(1, min(8, e))
    t = max(1, int(round(2 ** rng.uniform(0, math.log2(12000)))))
    bs = rng.choice([8, 16, 32, 48, 64])
    id_dtype = rng.choice([torch.int32, torch.int64])
    uniform = rng.random() < 0.3  # repeated and out-of-range ids instead of top-k routing
    with_map = rng.random() < 0.3
    if i % 10 == 9:  # more than 65536 routes: the multi-round one-workgroup kernel
        e, topk, t = max(e, 8), 8, rng.randint(8200, 12000)
    return e, topk, t, bs, id_dtype, uniform, with_map


ALIGN_CASES = [_align_case(i) for i in range(40)]


@pytest.mark.parametrize("i", range(len(ALIGN_CASES)))
def test_moe_align_random_shapes(i):
    """moe_align_block_size bit for bit against the oracle's stable order: 1-1024 experts,
    up to ~96K routes (the one-workgroup, many-workgroup and multi-round paths), every block
    size, int32 / int64 ids, ids outside [0, E) and expert maps with unmapped experts."""
    E, topk, T, bs, id_dtype, uniform, with_map = ALIGN_CASES[i]
    print(f"case align-sweep {i}: E={E} topk={topk} T={T} bs={bs} {id_dtype} uniform={uniform} "
          f"map={with_map}", flush=True)
    gen = torch.Generator().manual_seed(1200 + i)
    if uniform:
        ids = torch.randint(-1, E + 2, (T, topk), generator=gen)
    else:
        _, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    ids = ids.to(id_dtype)
    emap = None
    if with_map:
        emap = torch.randint(-1, E, (E,), generator=gen, dtype=torch.int32)
    numel = ids.numel()
    s = torch.empty(numel + E * (bs - 1), dtype=torch.int32, device="cuda")
    e = torch.empty(s.numel() // bs + 1, dtype=torch.int32, device="cuda")
    n = torch.empty(1, dtype=torch.int32, device="cuda")
    capi.moe_align_block_size(ids.cuda(), E, bs, s, e, n,
                              None if emap is None else emap.cuda())
    rs, re, rn = O.moe_align_block_size(ids.numpy(), E, bs,
                                        expert_map=None if emap is None else emap.numpy())
    assert int(n.cpu()[0]) == int(rn[0])
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy(), re)


def _layer_case(i):
    rng = random.Random(7800 + i)
    fmt = ("u4", "u4b8", "u8b128", "mxfp4", "nvfp4")[i % 5]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    e = rng.randint(2, 12)
    topk = rng.randint(1, min(4, e))
    t = max(1, int(round(2 ** rng.uniform(0, math.log2(400)))))
    h = 128 * rng.randint(1, 4)
    inter = 128 * rng.randint(1, 3)
    return fmt, dtype, e, topk, t, h, inter


LAYER_CASES = [_layer_case(i) for i in range(20)]


@pytest.mark.parametrize("i", range(len(LAYER_CASES)))
def test_fused_marlin_moe_random_layers(i):
    """fused_marlin_moe (align, stage 1, SiLU-gated activation, stage 2 with router weights,
    top-k sum; the block size from the reference's heuristic) against the oracle's per-token
    layer at random sizes, within twice the GEMM tolerance (two GEMMs in a row)."""
    from marlin_v100_amd.fused_marlin_moe import fused_marlin_moe

    fmt, dtype, E, topk, T, H, I = LAYER_CASES[i]
    print(f"case layer-sweep {i}: fmt={fmt} dtype={dtype} E={E} topk={topk} T={T} H={H} I={I}",
          flush=True)

    def experts(k, n, seed):
        cases = [make_case(fmt, k, n, dtype, seed=seed + j) for j in range(E)]
        words = torch.stack([capi.gptq_marlin_repack(c.gptq_words.cuda(), None, k, n, BITS[fmt])
                             for c in cases])
        scales = torch.stack([c.scales for c in cases]).cuda()
        zeros = (torch.stack([c.zeros for c in cases]).cuda()
                 if cases[0].zeros is not None else None)
        glob = (torch.cat([c.global_scale for c in cases]).cuda()
                if cases[0].global_scale is not None else None)
        return cases[0].type_id, words, scales, zeros, glob, torch.stack([c.deq for c in cases])

    tid, w13, s13, z13, g13, d13 = experts(H, 2 * I, 1000 + 37 * i)
    _, w2, s2, z2, g2, d2 = experts(I, H, 2000 + 37 * i)
    gen = torch.Generator().manual_seed(3000 + i)
    x = torch.randn((T, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    out = fused_marlin_moe(x.cuda(), w13, w2, None, None, s13, s2, tw.cuda(), ids.cuda(), tid,
                           global_scale1=g13, global_scale2=g2, w1_zeros=z13, w2_zeros=z2,
                           is_w1_zp_float=z13 is not None, is_w2_zp_float=z2 is not None).cpu()
    ref = O.moe_layer_ref(x, d13, d2, tw, ids)
    assert O.max_abs_rel_err(out, ref) <= 2 * TOL


def _large_moe_case(i):
    rng = random.Random(7900 + i)
    fmt = ("u4", "u4b8", "u8b128", "mxfp4", "nvfp4", "fp8")[i % 6]
    dtype = rng.choice([torch.float16, torch.bfloat16])
    e = rng.randint(4, 8)
    topk = rng.randint(2, 4)
    t = max(1, int(round(2 ** rng.uniform(2, math.log2(600)))))
    k = 128 * rng.randint(8, 24)
    n = 256 * rng.randint(4, 12)
    return fmt, dtype, e, topk, t, k, n


LARGE_MOE_CASES = [_large_moe_case(i) for i in range(12)]


@pytest.mark.parametrize("i", range(len(LARGE_MOE_CASES)))
def test_moe_gemm_random_large_shapes(i):
    """MoE GEMMs at larger K (1024-3072) and size_n (1024-3072) with up to 600 tokens: both
    the few-routes kernel (two waves per SIMD) and the multistage blocks at sizes near the
    production layer's, route by route against the oracle."""
    fmt, dtype, E, topk, T, K, N = LARGE_MOE_CASES[i]
    bs = 64 if T * topk > 16 * E else 16
    print(f"case moe-sweep-large {i}: fmt={fmt} dtype={dtype} E={E} topk={topk} T={T} K={K} "
          f"N={N} bs={bs}", flush=True)
    cases = [make_case(fmt, K, N, dtype, seed=1500 + 31 * i + j) for j in range(E)]
    words = torch.stack([capi.gptq_marlin_repack(c.gptq_words.cuda(), None, K, N, BITS[fmt])
                         for c in cases])
    scales = torch.stack([c.scales for c in cases]).cuda()
    zeros = torch.stack([c.zeros for c in cases]).cuda() if cases[0].zeros is not None else None
    glob = (torch.cat([c.global_scale for c in cases]).cuda()
            if cases[0].global_scale is not None else None)
    gen = torch.Generator().manual_seed(1600 + i)
    x = torch.randn((T, K), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    out = capi.moe_wna16_marlin_gemm(
        x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(), tw.cuda(), bs, topk, True,
        cases[0].type_id, T, N, K, b_zeros=zeros, global_scale=glob,
        is_zp_float=zeros is not None).cpu()
    flat = ids.reshape(-1)
    xr = x.float()[torch.arange(flat.numel()) // topk]
    ref = torch.empty((flat.numel(), N))
    for ex in range(E):
        rows = (flat == ex).nonzero().flatten()
        ref[rows] = xr[rows] @ cases[ex].deq.float()
    ref = ref * tw.reshape(-1, 1)
    assert O.max_abs_rel_err(out, ref) <= TOL
