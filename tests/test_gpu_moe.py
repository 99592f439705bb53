"""GPU parity of the MoE path: moe_align_block_size bit-exact against the stable-order
oracle (plus the KAT from the reference tests), each moe_wna16_marlin_gemm stage against
the oracle within 1e-2*max|ref|, and the full fused_marlin_moe layer (small shapes against
the oracle, the cfg5 shape at full size against the library's own dequantized experts)."""
import numpy as np
import pytest
import torch

import oracle as O
from marlin_v100_amd import capi
from tests.quant_cases import BITS, make_case

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _align(topk_ids, E, bs, expert_map=None):
    numel = topk_ids.numel()
    sorted_numel = numel + E * (bs - 1)
    s = torch.empty(sorted_numel, dtype=torch.int32, device="cuda")
    e = torch.empty(sorted_numel // bs + 1, dtype=torch.int32, device="cuda")
    n = torch.empty(1, dtype=torch.int32, device="cuda")
    capi.moe_align_block_size(topk_ids.cuda(), E, bs, s, e, n,
                              None if expert_map is None else expert_map.cuda())
    return s.cpu().numpy(), e.cpu().numpy(), n.cpu().numpy()


def test_moe_align_kat():
    # tests/test_marlin_moe.py:274-291
    ids = torch.tensor([[0, 3], [1, 3], [0, 2], [1, 0]], dtype=torch.int32)
    s, e, n = _align(ids, 4, 4)
    assert n[0] == 16
    assert s[:16].tolist() == [0, 4, 7, 8, 2, 6, 8, 8, 5, 8, 8, 8, 1, 3, 8, 8]
    assert e[:4].tolist() == [0, 1, 2, 3]
    assert (s[16:] == 8).all()


@pytest.mark.parametrize("tokens,E,topk,bs", [(16, 256, 8, 64), (2048, 256, 8, 64), (7, 8, 2, 16),
                                               (300, 64, 6, 8), (1000, 128, 4, 48),
                                               (3000, 512, 8, 32), (5000, 1024, 8, 16),
                                               (8192, 256, 8, 64), (9000, 256, 8, 64)])
@pytest.mark.parametrize("id_dtype", [torch.int32, torch.int64])
def test_moe_align_matches_oracle(tokens, E, topk, bs, id_dtype):
    gen = torch.Generator().manual_seed(tokens + E)
    logits = torch.randn((tokens, E), generator=gen)
    _, ids = O.route_topk(logits, topk)
    ids = ids.to(id_dtype)
    s, e, n = _align(ids, E, bs)
    rs, re, rn = O.moe_align_block_size(ids.numpy(), E, bs)
    assert n[0] == rn[0]
    assert np.array_equal(s, rs)
    assert np.array_equal(e, re)


def test_moe_align_expert_map_and_invalid_ids():
    E, bs = 16, 16
    gen = torch.Generator().manual_seed(1)
    ids = torch.randint(-2, E + 3, (50, 4), generator=gen, dtype=torch.int32)
    emap = torch.tensor([i // 2 if i % 3 else -1 for i in range(E)], dtype=torch.int32)
    s, e, n = _align(ids, E, bs, emap)
    rs, re, rn = O.moe_align_block_size(ids.numpy(), E, bs, expert_map=emap.numpy())
    assert n[0] == rn[0] and np.array_equal(s, rs) and np.array_equal(e, re)


def _make_experts(fmt, E, k, n, dtype, seed):
    cases = [make_case(fmt, k, n, dtype, seed=seed + i) for i in range(E)]
    bits = BITS[fmt]
    words = torch.stack([capi.gptq_marlin_repack(c.gptq_words.cuda(), None, k, n, bits)
                         for c in cases])
    scales = torch.stack([c.scales for c in cases]).cuda()
    zeros = torch.stack([c.zeros for c in cases]).cuda() if cases[0].zeros is not None else None
    glob = (torch.cat([c.global_scale for c in cases]).cuda()
            if cases[0].global_scale is not None else None)
    deq = torch.stack([c.deq for c in cases])
    return cases[0].type_id, words, scales, zeros, glob, deq


@pytest.mark.parametrize("fmt", ["u4", "u4b8", "u8b128", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs", [8, 16, 48, 64])
def test_moe_gemm_stage1(fmt, dtype, bs):
    T, E, topk, H, N = 37, 8, 3, 256, 512
    print(f"case fmt={fmt} dtype={dtype} bs={bs}", flush=True)
    tid, words, scales, zeros, glob, deq = _make_experts(fmt, E, H, N, dtype, 10)
    gen = torch.Generator().manual_seed(bs)
    x = torch.randn((T, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    out = capi.moe_wna16_marlin_gemm(x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(),
                                     tw.cuda(), bs, topk, False, tid, T, N, H, b_zeros=zeros,
                                     global_scale=glob, is_zp_float=zeros is not None).cpu()
    ref = torch.empty((T * topk, N))
    for r in range(T * topk):
        ref[r] = x[r // topk].float() @ deq[ids.reshape(-1)[r]].float()
    assert O.max_abs_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("T", [6, 96])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_moe_gemm_nvfp4_bias_under_router_weights(T, dtype):
    """NVFP4 with a bias and router weights: the bias is multiplied by the expert's global
    scale as passed to the op, then by the router weight, as the reference's MoE epilogue and
    bias init do (moe sm70_marlin_gemm.cuh:3490-3503, sm70_marlin_bias.cu:56-58); without
    router weights it is added as is.  T = 6 / 96: few-routes and multistage moe blocks."""
    E, topk, K, N, bs = 4, 2, 256, 256, 16
    tid, words, scales, _z, glob, deq = _make_experts("nvfp4", E, K, N, dtype, 30)
    gen = torch.Generator().manual_seed(31 + T)
    x = torch.randn((T, K), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    # scaled so that the bias term stays comparable with the product under either rule
    bias = (torch.randn((E, N), generator=gen) * 0.1 / glob.cpu().view(E, 1)).to(dtype)
    flat = ids.reshape(-1)
    for mul in (False, True):
        out = capi.moe_wna16_marlin_gemm(
            x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(), tw.cuda(), bs, topk, mul,
            tid, T, N, K, global_scale=glob, b_bias=O.marlin_permute_bias(bias).cuda()).cpu()
        ref = torch.empty((flat.numel(), N))
        for r in range(flat.numel()):
            ex = int(flat[r])
            v = x[r // topk].float() @ deq[ex].float()
            if mul:
                ref[r] = (v + bias[ex].float() * float(glob[ex])) * tw.reshape(-1)[r]
            else:
                ref[r] = v + bias[ex].float()
        assert O.max_abs_rel_err(out, ref) <= TOL, mul


@pytest.mark.parametrize("bs", [8, 16, 64])
@pytest.mark.parametrize("fmt", ["u4", "mxfp4"])
def test_moe_gemm_every_route_on_its_own_expert(bs, fmt):
    """Fewer routes than experts, each route on a different expert: every route is a moe
    block of its own, exactly as many blocks as the launch bound allows (routes + routes x
    (bs - 1)) / bs, so a bound one block short would drop the last route."""
    T, E, topk, H, N = 4, 64, 8, 256, 256
    tid, words, scales, zeros, glob, deq = _make_experts(fmt, E, H, N, torch.bfloat16, 60)
    gen = torch.Generator().manual_seed(61)
    x = torch.randn((T, H), generator=gen).bfloat16()
    ids = torch.randperm(E, generator=gen)[: T * topk].to(torch.int32).reshape(T, topk)
    tw = torch.rand((T, topk), generator=gen)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    assert int(npad[0]) == T * topk * bs
    out = capi.moe_wna16_marlin_gemm(x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(),
                                     tw.reshape(-1).cuda(), bs, topk, False, tid, T, N, H,
                                     b_zeros=zeros, global_scale=glob,
                                     is_zp_float=zeros is not None).cpu()
    ref = torch.empty((T * topk, N))
    for r in range(T * topk):
        ref[r] = x[r // topk].float() @ deq[ids.reshape(-1)[r]].float()
    assert O.max_abs_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_moe_gemm_stage2_topk_weights_and_bias(dtype):
    T, E, topk, K, N, bs = 23, 8, 2, 256, 256, 16
    tid, words, scales, zeros, glob, deq = _make_experts("u4", E, K, N, dtype, 20)
    gen = torch.Generator().manual_seed(5)
    x = torch.randn((T * topk, K), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    bias = (torch.randn((E, N), generator=gen) * 0.1).to(dtype)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    out = capi.moe_wna16_marlin_gemm(x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(),
                                     tw.cuda(), bs, 1, True, tid, T * topk, N, K, b_zeros=zeros,
                                     b_bias=O.marlin_permute_bias(bias).cuda(),
                                     is_zp_float=True).cpu()
    flat = ids.reshape(-1)
    ref = torch.empty((T * topk, N))
    for r in range(T * topk):
        ref[r] = (x[r].float() @ deq[flat[r]].float() + bias[flat[r]].float()) * tw.reshape(-1)[r]
    assert O.max_abs_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_marlin_moe_layer(dtype):
    from marlin_v100_amd.fused_marlin_moe import fused_marlin_moe

    T, E, topk, H, I = 33, 16, 4, 256, 128
    tid, w13, s13, z13, _, d13 = _make_experts("u4", E, H, 2 * I, dtype, 30)
    _, w2, s2, z2, _, d2 = _make_experts("u4", E, I, H, dtype, 60)
    gen = torch.Generator().manual_seed(8)
    x = torch.randn((T, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    out = fused_marlin_moe(x.cuda(), w13, w2, None, None, s13, s2, tw.cuda(), ids.cuda(), tid,
                           w1_zeros=z13, w2_zeros=z2, is_w1_zp_float=True,
                           is_w2_zp_float=True).cpu()
    ref = O.moe_layer_ref(x, d13, d2, tw, ids)
    assert O.max_abs_rel_err(out, ref) <= 2 * TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,d", [(64, 1536), (7, 24), (5, 12), (0, 16)])
def test_silu_and_mul(dtype, rows, d):
    """Native activation vs the reference expression F.silu(gate) * up in the element type
    (activation.py:45-52): silu rounded to the element type, then the product."""
    gen = torch.Generator().manual_seed(rows * 131 + d)
    x = (torch.randn((rows, 2 * d), generator=gen) * 3).to(dtype)
    out = torch.empty((rows, d), dtype=dtype, device="cuda")
    capi.silu_and_mul(out, x.cuda())
    g, u = x[:, :d].float(), x[:, d:].float()
    ref = (torch.nn.functional.silu(g).to(dtype).float() * u).to(dtype)
    got = out.cpu()
    if rows == 0:
        return
    assert O.max_abs_rel_err(got, ref) <= 1e-2
    exact = (got.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert exact >= 0.99, exact


@pytest.mark.parametrize("T", [16, 2048])
def test_fused_marlin_moe_baseline_shape(T):
    """cfg5 at full size (E=256, top-8, H=3072, I=1536, uint4 + float zp g128, bf16): the
    few-routes kernel (T=16) and the multistage MoE blocks (T=2048) against an fp32 layer
    built from the library's dequantized experts (the dequantize op is bit-exact against the
    oracle in test_gpu_repack_dequant.py), on 24 tokens spread over the batch."""
    import bench
    from marlin_v100_amd.fused_marlin_moe import fused_marlin_moe
    from marlin_v100_amd.scalar_type import scalar_types

    E, topk, H, I = 256, 8, 3072, 1536
    dt = torch.bfloat16
    print(f"case cfg5 T={T}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(T)
    w13 = [bench.make_weights("u4", H, 2 * I, dt, gen) for _ in range(E)]
    w2 = [bench.make_weights("u4", I, H, dt, gen) for _ in range(E)]
    q13 = torch.stack([w["qweight"] for w in w13]); s13 = torch.stack([w["scales"] for w in w13])
    z13 = torch.stack([w["zeros"] for w in w13])
    q2 = torch.stack([w["qweight"] for w in w2]); s2 = torch.stack([w["scales"] for w in w2])
    z2 = torch.stack([w["zeros"] for w in w2])
    x = torch.randn((T, H), generator=gen, device="cuda").to(dt)
    tw, ids = torch.topk(torch.softmax(torch.randn((T, E), generator=gen, device="cuda"), -1),
                         topk, -1)
    tw = (tw / tw.sum(-1, keepdim=True)).float().contiguous()
    ids = ids.to(torch.int32).contiguous()
    qid = scalar_types.uint4.id
    out = fused_marlin_moe(x, q13, q2, None, None, s13, s2, tw, ids, qid, w1_zeros=z13,
                           w2_zeros=z2, is_w1_zp_float=True, is_w2_zp_float=True)
    tokens = torch.unique(torch.linspace(0, T - 1, 24).long()).tolist()
    ref = torch.zeros((len(tokens), H), device="cuda")
    for j, t in enumerate(tokens):
        xt = x[t].float()[None]
        for r in range(topk):
            e = int(ids[t, r])
            d13 = capi.dequantize(q13[e], s13[e], qid, H, 2 * I, dt, b_zeros=z13[e]).float()
            h = xt @ d13
            act = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
            d2 = capi.dequantize(q2[e], s2[e], qid, I, H, dt, b_zeros=z2[e]).float()
            ref[j] += float(tw[t, r]) * (act @ d2)[0]
    assert O.max_abs_rel_err(out[tokens].float().cpu(), ref.cpu()) <= 2 * TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("topk", [1, 2, 3, 4, 6, 8])
@pytest.mark.parametrize("tokens,hidden", [(33, 3072), (5, 100), (1, 8), (0, 64)])
def test_moe_sum(dtype, topk, tokens, hidden):
    """Native moe_sum bit-exact against the reference's arithmetic (per-addition rounding
    for top-k 2..4, one fp32 rounding otherwise); hidden 3072 and 8 take the 16-byte path,
    100 the element path."""
    gen = torch.Generator().manual_seed(tokens * 7 + topk)
    x = (torch.randn((tokens, topk, hidden), generator=gen) * 4).to(dtype)
    out = torch.empty((tokens, hidden), dtype=dtype, device="cuda")
    capi.moe_sum(x.cuda(), out)
    assert torch.equal(out.cpu(), O.moe_sum(x))
    if topk == 3 and dtype == torch.bfloat16 and tokens > 0:
        kat = torch.zeros((1, 3, hidden), dtype=dtype)
        kat[0, 0], kat[0, 1], kat[0, 2] = 1.0, 2.0 ** -8, 2.0 ** -8
        o = torch.empty((1, hidden), dtype=dtype, device="cuda")
        capi.moe_sum(kat.cuda(), o)
        assert (o.cpu() == 1.0).all()


def _moe_ref(x, deq, ids, topk, tw=None, mul=False):
    """fp32 oracle per route: row r uses token r // topk and expert ids.flat[r]."""
    flat = ids.reshape(-1)
    ref = torch.empty((flat.numel(), deq.shape[-1]))
    for r in range(flat.numel()):
        ref[r] = x[r // topk].float() @ deq[flat[r]].float()
        if mul:
            ref[r] *= tw.reshape(-1)[r]
    return ref


@pytest.mark.parametrize("fmt", ["u4", "u4b8", "u8b128"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs", [16, 32, 48, 64])
def test_moe_gemm_multistage_integer(fmt, dtype, bs):
    """More than 16 routes per expert on average (T * top_k > 16 * E): the multistage MoE
    blocks with integer weights, every route against the oracle's dequantized experts."""
    T, E, topk, H, N = 96, 4, 2, 256, 512
    print(f"case moe-multistage fmt={fmt} dtype={dtype} bs={bs}", flush=True)
    tid, words, scales, zeros, glob, deq = _make_experts(fmt, E, H, N, dtype, 40)
    gen = torch.Generator().manual_seed(bs + 7)
    x = torch.randn((T, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    for mul in (False, True):
        out = capi.moe_wna16_marlin_gemm(x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(),
                                         tw.cuda(), bs, topk, mul, tid, T, N, H, b_zeros=zeros,
                                         global_scale=glob, is_zp_float=zeros is not None).cpu()
        assert O.max_abs_rel_err(out, _moe_ref(x, deq, ids, topk, tw, mul)) <= TOL


@pytest.mark.parametrize("fmt", ["u4", "u4b8", "u8b128"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,E,topk,bs,H", [
    (600, 4, 2, 16, 256),    # 19 moe blocks per expert
    (600, 4, 2, 64, 256),    # 5 moe blocks per expert
    (2200, 2, 1, 16, 256),   # runs of more than 64 moe blocks of one expert
    (160, 4, 2, 32, 1024),   # 8 K steps: split K
    (96, 3, 2, 64, 288),     # a 32-deep K tail (channelwise uint8b128 only)
    (300, 4, 2, 64, 768),    # K % 384 == 0 with three 256-column blocks: the column walk
    (300, 4, 2, 16, 1152),
])
def test_moe_gemm_many_blocks_per_expert(fmt, dtype, T, E, topk, bs, H):
    """The multistage MoE kernel with many consecutive moe blocks per expert, split K and a
    K tail; every route (with its router weight) against the oracle."""
    if fmt != "u8b128" and H % 128:
        pytest.skip("128-deep groups need K % 128 == 0")
    N = 768 if H % 384 == 0 else 256
    print(f"case moe-blocks fmt={fmt} dtype={dtype} T={T} E={E} topk={topk} bs={bs} H={H}",
          flush=True)
    tid, words, scales, zeros, glob, deq = _make_experts(fmt, E, H, N, dtype, 60)
    gen = torch.Generator().manual_seed(T + bs + H)
    x = torch.randn((T, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    out = capi.moe_wna16_marlin_gemm(x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(),
                                     tw.cuda(), bs, topk, True, tid, T, N, H, b_zeros=zeros,
                                     global_scale=glob, is_zp_float=zeros is not None).cpu()
    assert O.max_abs_rel_err(out, _moe_ref(x, deq, ids, topk, tw, True)) <= TOL


@pytest.mark.parametrize("fmt", ["u4", "u4b8", "u8b128"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,E,topk,bs,K,N,skew", [
    (5, 8, 2, 16, 384, 256, False),     # three K steps
    (12, 4, 3, 64, 768, 320, False),    # five 64-column groups
    (40, 8, 2, 64, 1152, 256, True),    # one expert takes ~40 routes: several 16-row parts
    (3, 256, 8, 64, 384, 128, False),   # many experts, most blocks empty
    (7, 8, 1, 8, 1536, 192, False),     # 8-row moe blocks
    (30, 16, 4, 32, 3072, 128, True),
])
def test_moe_gemm_few_routes_parts_and_bias(fmt, dtype, T, E, topk, bs, K, N, skew):
    """The few-routes MoE kernel (one wave per moe block x 64-column group) at K = 384 ..
    3072, on blocks with several 16-row parts holding routes (skewed routing), many empty
    experts and 8-row blocks: every route, with and without its router weight (and a bias),
    against the oracle."""
    print(f"case moe-few fmt={fmt} dtype={dtype} T={T} E={E} topk={topk} bs={bs} K={K} N={N}",
          flush=True)
    assert T * topk <= 16 * E  # the few-routes plan
    tid, words, scales, zeros, glob, deq = _make_experts(fmt, E, K, N, dtype, 70)
    gen = torch.Generator().manual_seed(T + E + K)
    x = torch.randn((T, K), generator=gen).to(dtype)
    logits = torch.randn((T, E), generator=gen)
    if skew:
        logits[:, 0] += 6.0
    tw, ids = O.route_topk(logits, topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    bias = (torch.randn((E, N), generator=gen) * 0.1).to(dtype)
    flat = ids.reshape(-1)
    for mul, with_bias in ((False, False), (True, True)):
        out = capi.moe_wna16_marlin_gemm(
            x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(), tw.cuda(), bs, topk, mul,
            tid, T, N, K, b_zeros=zeros, global_scale=glob, is_zp_float=zeros is not None,
            b_bias=O.marlin_permute_bias(bias).cuda() if with_bias else None).cpu()
        ref = torch.empty((flat.numel(), N))
        for r in range(flat.numel()):
            v = x[r // topk].float() @ deq[flat[r]].float()
            if with_bias:
                v = v + bias[flat[r]].float()
            ref[r] = v * tw.reshape(-1)[r] if mul else v
        assert O.max_abs_rel_err(out, ref) <= TOL, (mul, with_bias)


@pytest.mark.parametrize("fmt", ["u4", "u8b128", "mxfp4", "nvfp4"])
@pytest.mark.parametrize("n", [320, 384])
@pytest.mark.parametrize("T,bs", [(5, 16), (96, 16), (96, 48), (96, 64)])
def test_moe_gemm_size_n_multiple_of_64(fmt, n, T, bs):
    """size_n % 256 != 0 (the reference accepts size_n % 64, ops.cu:390-392): 64- and
    128-column blocks of the multistage kernel, and the few-routes kernel."""
    E, topk, H = 4, 2, 256
    dtype = torch.bfloat16
    print(f"case moe-narrow fmt={fmt} n={n} T={T} bs={bs}", flush=True)
    tid, words, scales, zeros, glob, deq = _make_experts(fmt, E, H, n, dtype, 50)
    gen = torch.Generator().manual_seed(T + bs)
    x = torch.randn((T, H), generator=gen).to(dtype)
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    s, e, npad = (torch.from_numpy(v) for v in O.moe_align_block_size(ids.numpy(), E, bs))
    out = capi.moe_wna16_marlin_gemm(x.cuda(), words, scales, s.cuda(), e.cuda(), npad.cuda(),
                                     tw.cuda(), bs, topk, False, tid, T, n, H, b_zeros=zeros,
                                     global_scale=glob, is_zp_float=zeros is not None).cpu()
    assert O.max_abs_rel_err(out, _moe_ref(x, deq, ids, topk)) <= TOL


@pytest.mark.parametrize("topk", [1, 3, 4, 8])
def test_moe_sum_fp32(topk):
    gen = torch.Generator().manual_seed(topk)
    x = torch.randn((37, topk, 200), generator=gen)
    out = torch.empty((37, 200), device="cuda")
    capi.moe_sum(x.cuda(), out)
    ref = x[:, 0].clone()
    for j in range(1, topk):
        ref += x[:, j]  # fp32 additions in index order
    assert torch.equal(out.cpu(), ref)


def test_moe_sum_many_tokens():
    """More than 65535 tokens in one call (no grid-dimension limit), odd hidden size."""
    tokens, topk, hidden = 70001, 2, 3
    gen = torch.Generator().manual_seed(9)
    x = torch.randn((tokens, topk, hidden), generator=gen).to(torch.bfloat16)
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device="cuda")
    capi.moe_sum(x.cuda(), out)
    assert torch.equal(out.cpu(), O.moe_sum(x))


def test_fused_marlin_moe_reference_keywords():
    """The reference's keyword set (fused_marlin_moe.py:217-255): activation, moe_sum,
    workspace, intermediate caches, output, is_k_full, input_dtype, inplace; a custom
    activation callback; act-order arguments raise NotImplementedError."""
    from marlin_v100_amd import _custom_ops as cops
    from marlin_v100_amd.fused_marlin_moe import (MoEActivation, apply_moe_activation,
                                                  fused_marlin_moe)

    T, E, topk, H, I = 17, 8, 2, 256, 128
    dtype = torch.bfloat16
    tid, w13, s13, z13, _, d13 = _make_experts("u4", E, H, 2 * I, dtype, 70)
    _, w2, s2, z2, _, d2 = _make_experts("u4", E, I, H, dtype, 90)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn((T, H), generator=gen).to(dtype).cuda()
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    tw, ids = tw.cuda(), ids.cuda()
    ref = O.moe_layer_ref(x.cpu(), d13, d2, tw.cpu(), ids.cpu())
    cache13 = torch.empty((T * topk * max(2 * I, H),), dtype=dtype, device="cuda")
    cache2 = torch.empty((T * topk, I), dtype=dtype, device="cuda")
    out = torch.empty((T, H), dtype=dtype, device="cuda")
    got = fused_marlin_moe(
        hidden_states=x, w1=w13, w2=w2, bias1=None, bias2=None, w1_scale=s13, w2_scale=s2,
        topk_weights=tw, topk_ids=ids, quant_type_id=tid, apply_router_weight_on_input=False,
        global_num_experts=-1, activation=MoEActivation.SILU, moe_sum=cops.moe_sum,
        expert_map=None, global_scale1=None, global_scale2=None, g_idx1=None, g_idx2=None,
        sort_indices1=None, sort_indices2=None, w1_zeros=z13, w2_zeros=z2, is_w1_zp_float=True,
        is_w2_zp_float=True, workspace=None, intermediate_cache13=cache13,
        intermediate_cache2=cache2, is_k_full=True, output=out, input_dtype=None, inplace=False)
    assert O.max_abs_rel_err(out.cpu(), ref) <= 2 * TOL
    calls = []

    def act(a, o, i):
        calls.append(a)
        apply_moe_activation(a, o, i)

    got2 = fused_marlin_moe(x, w13, w2, None, None, s13, s2, tw, ids, tid, False, -1,
                            MoEActivation.SILU, act, w1_zeros=z13, w2_zeros=z2,
                            is_w1_zp_float=True, is_w2_zp_float=True)
    assert calls == [MoEActivation.SILU]
    assert O.max_abs_rel_err(got2.cpu(), ref) <= 2 * TOL
    with pytest.raises(NotImplementedError):
        fused_marlin_moe(x, w13, w2, None, None, s13, s2, tw, ids, tid,
                         g_idx1=torch.zeros(H, dtype=torch.int32, device="cuda"),
                         w1_zeros=z13, w2_zeros=z2, is_w1_zp_float=True, is_w2_zp_float=True)


@pytest.mark.parametrize("fmt", ["u4", "u4b8", "u8b128", "nvfp4"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs", [16, 32, 48, 64])
@pytest.mark.parametrize("bias,mul", [(False, False), (True, True)])
def test_moe_stage1_silu_fused_is_bit_exact(fmt, dtype, bs, bias, mul):
    """marlin_moe_wna16_marlin_gemm_silu == marlin_moe_wna16_marlin_gemm then silu_and_mul,
    bit for bit (the fused epilogue rounds the stage-1 outputs as the store would, then applies
    the same silu_mul); the two-pass path itself is checked against the oracle above."""
    E, T, topk, K, I = 4, 96, 2, 256, 256
    if fmt == "nvfp4" and bs >= 48:
        pytest.skip("small-group metadata of 48/64-row blocks takes the tiled kernel (not fused)")
    print(f"case fused-silu fmt={fmt} dtype={dtype} bs={bs} bias={bias} mul={mul}", flush=True)
    tid, words, scales, zeros, glob, _deq = _make_experts(fmt, E, K, 2 * I, dtype, 700 + bs)
    gen = torch.Generator().manual_seed(bs)
    x = torch.randn((T, K), generator=gen).to(dtype).cuda()
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    numel = ids.numel()
    s = torch.empty(numel + E * (bs - 1), dtype=torch.int32, device="cuda")
    e = torch.empty(s.numel() // bs + 1, dtype=torch.int32, device="cuda")
    npad = torch.empty(1, dtype=torch.int32, device="cuda")
    capi.moe_align_block_size(ids.cuda(), E, bs, s, e, npad)
    b = (torch.randn((E, 2 * I), generator=gen) * 0.1).to(dtype).cuda() if bias else None
    kw = dict(b_bias=b, global_scale=glob, b_zeros=zeros, is_zp_float=zeros is not None)
    args = (x, words, scales, s, e, npad, tw.cuda(), bs, topk, mul, tid, T, 2 * I, K)
    h = capi.moe_wna16_marlin_gemm(*args, **kw)
    ref = torch.empty((T * topk, I), dtype=dtype, device="cuda")
    capi.silu_and_mul(ref, h)
    out = torch.full((T * topk, I), float("nan"), dtype=dtype, device="cuda")
    capi.moe_wna16_marlin_gemm(*args, c=out, silu_gated=True, **kw)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("fmt", ["u4", "u4b8", "u8b128", "fp8"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bias,mul", [(False, False), (True, True)])
def test_moe_stage1_silu_fused_decode_batches_bit_exact(fmt, dtype, bias, mul):
    """Few routes per expert take the decode kernel, whose fused form gives each wave two gate
    and the two matching up tiles: same bits as stage 1 then silu_and_mul.  K = 640 is five
    steps (one full trip of the three-deep ring and two after it); I = 192 is not a multiple
    of 128 columns."""
    E, T, topk, K, I, bs = 16, 8, 2, 640, 192, 16
    print(f"case fused-silu-decode fmt={fmt} dtype={dtype} bias={bias} mul={mul}", flush=True)
    tid, words, scales, zeros, glob, _d = _make_experts(fmt, E, K, 2 * I, dtype, 40)
    gen = torch.Generator().manual_seed(41)
    ids = torch.randint(0, E, (T, topk), generator=gen, dtype=torch.int32)
    tw = torch.rand((T, topk), generator=gen)
    s = torch.empty(ids.numel() + E * (bs - 1), dtype=torch.int32, device="cuda")
    e = torch.empty(s.numel() // bs + 1, dtype=torch.int32, device="cuda")
    npad = torch.empty(1, dtype=torch.int32, device="cuda")
    capi.moe_align_block_size(ids.cuda(), E, bs, s, e, npad)
    x = torch.randn((T, K), generator=gen).to(dtype).cuda()
    b = (torch.randn((E, 2 * I), generator=gen) * 0.1).to(dtype).cuda() if bias else None
    kw = dict(b_bias=b, global_scale=glob, b_zeros=zeros, is_zp_float=zeros is not None)
    args = (x, words, scales, s, e, npad, tw.reshape(-1).cuda(), bs, topk, mul, tid, T, 2 * I, K)
    h = capi.moe_wna16_marlin_gemm(*args, **kw)
    ref = torch.empty((T * topk, I), dtype=dtype, device="cuda")
    capi.silu_and_mul(ref, h)
    out = torch.full((T * topk, I), float("nan"), dtype=dtype, device="cuda")
    capi.moe_wna16_marlin_gemm(*args, c=out, silu_gated=True, **kw)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_moe_stage1_silu_fused_declines_tiled_plans():
    """A plan with no fused form (fp4 small-group metadata in 64-row moe blocks takes the
    tiled kernel) reports NOT_SUPPORTED and launches nothing (fused_marlin_moe then runs two
    passes)."""
    E, T, topk, K, I, bs = 4, 8, 2, 256, 256, 64
    tid, words, scales, zeros, glob, _d = _make_experts("nvfp4", E, K, 2 * I, torch.bfloat16, 5)
    ids = torch.randint(0, E, (T, topk), dtype=torch.int32)
    s = torch.empty(ids.numel() + E * (bs - 1), dtype=torch.int32, device="cuda")
    e = torch.empty(s.numel() // bs + 1, dtype=torch.int32, device="cuda")
    npad = torch.empty(1, dtype=torch.int32, device="cuda")
    capi.moe_align_block_size(ids.cuda(), E, bs, s, e, npad)
    x = torch.randn((T, K)).bfloat16().cuda()
    out = torch.full((T * topk, I), 7.0, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(capi.MarlinError) as err:
        capi.moe_wna16_marlin_gemm(x, words, scales, s, e, npad, torch.ones(T * topk).cuda(), bs,
                                   topk, False, tid, T, 2 * I, K, c=out, global_scale=glob,
                                   silu_gated=True)
    assert err.value.status == capi.STATUS_NOT_SUPPORTED
    torch.cuda.synchronize()
    assert (out == 7.0).all()


def test_fused_marlin_moe_fuse_activation_matches_two_pass():
    """fused_marlin_moe(fuse_activation=True) gives the two-pass layer's bits, for a batch
    large enough for the multistage kernel and for a decode-sized one."""
    from marlin_v100_amd.fused_marlin_moe import fused_marlin_moe

    T, E, topk, H, I = 200, 8, 2, 256, 128
    dtype = torch.bfloat16
    tid, w13, s13, z13, _, _d13 = _make_experts("u4", E, H, 2 * I, dtype, 90)
    _, w2, s2, z2, _, _d2 = _make_experts("u4", E, I, H, dtype, 91)
    gen = torch.Generator().manual_seed(92)
    x = torch.randn((T, H), generator=gen).to(dtype).cuda()
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), topk)
    kw = dict(w1_zeros=z13, w2_zeros=z2, is_w1_zp_float=True, is_w2_zp_float=True)
    two = fused_marlin_moe(x, w13, w2, None, None, s13, s2, tw.cuda(), ids.cuda(), tid, **kw)
    one = fused_marlin_moe(x, w13, w2, None, None, s13, s2, tw.cuda(), ids.cuda(), tid,
                           fuse_activation=True, **kw)
    assert torch.equal(one.view(torch.int16), two.view(torch.int16))
    # a decode-sized batch (few-routes kernel's fused form): same bits as two passes
    xs, tws, idss = x[:6].contiguous(), tw[:6].cuda(), ids[:6].cuda()
    fused = fused_marlin_moe(xs, w13, w2, None, None, s13, s2, tws, idss, tid,
                             fuse_activation=True, **kw)
    unfused = fused_marlin_moe(xs, w13, w2, None, None, s13, s2, tws, idss, tid, **kw)
    assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16))
