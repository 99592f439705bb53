"""GPU parity of the MoE router (topk_softmax / topk_sigmoid) against the CPU oracle, through
the C ABI and the torch ops: the reference test's known answer (tests/test_marlin_moe.py:248-272),
the tie rule, every gating dtype and id dtype, expert counts from 4 to 4096, and the BASELINE
cfg5 routing (T = 2048, E = 256, top-8, renormalized) at full size.

Ids are compared exactly wherever the oracle's choice scores of neighbouring ranks differ by
more than 1e-6 (otherwise the kernel's float32 exp and the oracle's may order a near-tie
differently); every row's chosen scores must match the oracle's within 2e-6.  Weights: within
rtol 1e-5 / atol 1e-6 of the oracle's float32 scores (the reference test allows 1e-4)."""
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from marlin_v100_amd import capi

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _oracle_scores(gating, bias, scoring):
    x = gating.float().numpy()
    if scoring == "softmax":
        ex = np.exp(x - x.max(axis=1, keepdims=True), dtype=np.float32)
        s = ex / ex.sum(axis=1, keepdims=True, dtype=np.float32)
    else:
        s = np.float32(1.0) / (np.float32(1.0) + np.exp(-x, dtype=np.float32))
    return s.astype(np.float32), (s if bias is None else s + bias.numpy()).astype(np.float32)


def _check(gating, k, renorm, bias, scoring, w, ids, tei):
    T = gating.shape[0]
    ref_w, ref_ids, ref_tei = O.topk_gating(gating.float().numpy(), k, renorm,
                                            None if bias is None else bias.numpy(), scoring)
    ids = ids.cpu().to(torch.int64).numpy() if ids.dtype != torch.uint32 else \
        ids.cpu().view(torch.int32).to(torch.int64).numpy()
    assert np.array_equal(tei.cpu().numpy(), ref_tei)
    scores, choice = _oracle_scores(gating, bias, scoring)
    exact_rows = 0
    for r in range(T):
        assert len(set(ids[r].tolist())) == k, f"row {r}: repeated expert"
        assert ids[r].min() >= 0 and ids[r].max() < gating.shape[1]
        np.testing.assert_allclose(choice[r, ids[r]], choice[r, ref_ids[r]], rtol=0, atol=2e-6)
        ranked = np.sort(choice[r])[::-1][:k + 1]
        if np.all(np.abs(np.diff(ranked)) > 1e-6):
            assert ids[r].tolist() == ref_ids[r].tolist(), f"row {r}"
            exact_rows += 1
    # weights: the oracle's scores at the kernel's ids (identical ids on all clear rows)
    ws = np.take_along_axis(scores, ids, 1)
    if renorm:
        s = ws.sum(axis=1, keepdims=True)
        ws = ws / np.where(s > 0, s, 1.0)
    np.testing.assert_allclose(w.cpu().numpy(), ws, rtol=1e-5, atol=1e-6)
    return exact_rows


def test_topk_softmax_reference_kat():
    with open(os.path.join(GOLDEN, "topk_softmax_kat.json")) as f:
        g = json.load(f)
    gating = torch.tensor(g["gating_fp16_values"], dtype=torch.float16).cuda()
    bias = torch.tensor(g["bias"], dtype=torch.float32).cuda()
    w, ids, tei = capi.topk_gating(gating, g["topk"], g["renormalize"], bias)
    assert ids.cpu().tolist() == g["topk_ids"]
    assert tei.cpu().tolist() == g["token_expert_indices"]
    np.testing.assert_allclose(w.cpu().numpy(), np.asarray(g["topk_weights"]), rtol=0, atol=1e-6)
    # the same through the registered torch op (reference wrapper shape)
    from marlin_v100_amd import _custom_ops as ops
    w2 = torch.empty_like(w)
    ids2 = torch.empty_like(ids)
    tei2 = torch.empty_like(tei)
    ops.topk_softmax(w2, ids2, tei2, gating, True, bias)
    assert torch.equal(ids2, ids) and torch.equal(tei2, tei) and torch.equal(w2, w)


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_topk_tie_rule(scoring):
    # equal inputs give bit-identical scores: the lower expert index wins every tie
    g = torch.zeros((3, 300), dtype=torch.bfloat16)
    g[1, ::7] = 1.0
    g[2, 200:] = 2.0
    w, ids, _ = capi.topk_gating(g.cuda(), 8, False, None, scoring)
    ids = ids.cpu().tolist()
    assert ids[0] == list(range(8))
    assert ids[1] == [0, 7, 14, 21, 28, 35, 42, 49]
    assert ids[2] == list(range(200, 208))
    ref_w, ref_ids, _ = O.topk_gating(g.float().numpy(), 8, False, None, scoring)
    assert ref_ids.tolist() == ids
    np.testing.assert_allclose(w.cpu().numpy(), ref_w, rtol=1e-6)


CASES = [(5, 4, 2), (33, 60, 6), (7, 128, 1), (16, 256, 8), (9, 384, 8), (3, 1000, 4),
         (64, 64, 64), (4, 2048, 32), (2, 4096, 256)]


@pytest.mark.parametrize("T,E,k", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_topk_matches_oracle(T, E, k, dtype, scoring):
    gen = torch.Generator().manual_seed(T * 131 + E + k)
    gating = (torch.randn((T, E), generator=gen) * 2).to(dtype)
    for renorm, use_bias in ((False, False), (True, False), (True, True)):
        bias = (torch.randn(E, generator=gen) * 0.05) if use_bias else None
        w, ids, tei = capi.topk_gating(gating.cuda(), k, renorm,
                                       None if bias is None else bias.cuda(), scoring)
        _check(gating, k, renorm, bias, scoring, w, ids, tei)


@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.uint32])
def test_topk_id_dtypes(ids_dtype):
    gen = torch.Generator().manual_seed(7)
    gating = torch.randn((40, 256), generator=gen)
    w32, ids32, tei32 = capi.topk_gating(gating.cuda(), 8, True)
    w, ids, tei = capi.topk_gating(gating.cuda(), 8, True, ids_dtype=ids_dtype)
    got = ids.cpu().view(torch.int32) if ids_dtype == torch.uint32 else ids.cpu()
    assert got.to(torch.int64).tolist() == ids32.cpu().to(torch.int64).tolist()
    assert torch.equal(w, w32) and torch.equal(tei, tei32)


def test_topk_no_tokens_and_op_errors():
    w, ids, tei = capi.topk_gating(torch.empty((0, 64), device="cuda"), 4)
    assert w.shape == (0, 4)
    from marlin_v100_amd import _custom_ops as ops
    g = torch.randn((4, 8), device="cuda")
    w = torch.empty((4, 2), device="cuda")
    ids = torch.empty((4, 2), dtype=torch.int32, device="cuda")
    tei = torch.empty((4, 2), dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="bias size mismatch, expected: 8"):
        ops.topk_softmax(w, ids, tei, g, False, torch.zeros(7, device="cuda"))
    with pytest.raises(RuntimeError, match="bias tensor must be float32"):
        ops.topk_sigmoid(w, ids, tei, g, False, torch.zeros(8, device="cuda").half())


def test_topk_baseline_routing_full_size():
    # BASELINE cfg5 router: logits [2048, 256] ~ N(0, 1), softmax top-8, renormalized
    gen = torch.Generator().manual_seed(1005)
    logits = torch.randn((2048, 256), generator=gen)
    w, ids, tei = capi.topk_gating(logits.cuda(), 8, True)
    exact = _check(logits, 8, True, None, "softmax", w, ids, tei)
    assert exact >= 0.95 * 2048  # rows without a 1e-6 near-tie among the top 9
    np.testing.assert_allclose(w.sum(dim=1).cpu().numpy(), 1.0, rtol=2e-6)


# ---- grouped_topk ------------------------------------------------------------------------

def test_grouped_topk_reference_kat():
    with open(os.path.join(GOLDEN, "grouped_topk_kat.json")) as f:
        g = json.load(f)
    scores = torch.tensor(g["scores"], dtype=torch.float32).cuda()
    bias = torch.tensor(g["bias"], dtype=torch.float32).cuda()
    args = (g["num_expert_group"], g["topk_group"], g["topk"], g["renormalize"],
            g["routed_scaling_factor"])
    vals, ids = capi.grouped_topk(scores, *args, bias, g["scoring_func"])
    assert ids.cpu().tolist() == g["topk_ids"]
    np.testing.assert_allclose(vals.cpu().numpy(), np.asarray(g["topk_weights"]), rtol=0,
                               atol=1e-6)
    from marlin_v100_amd import _custom_ops as ops
    vals2, ids2 = ops.grouped_topk(scores, *args, bias, g["scoring_func"])
    assert torch.equal(ids2, ids) and torch.equal(vals2, vals)


GROUPED = [  # (T, E, n_group, topk_group, topk)
    (16, 256, 8, 4, 8),      # DeepSeek-V3 shape
    (33, 64, 8, 3, 6), (7, 96, 4, 2, 5), (5, 160, 32, 4, 4), (9, 1024, 16, 4, 32),
    (4, 512, 1, 1, 22), (3, 8, 8, 8, 8), (2048, 256, 8, 4, 8),
    (6, 128, 8, 2, 6), (5, 512, 32, 8, 16),  # 16 experts per group
]


@pytest.mark.parametrize("T,E,ng,tg,k", GROUPED)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scoring", [0, 1])
def test_grouped_topk_matches_oracle(T, E, ng, tg, k, dtype, scoring):
    gen = torch.Generator().manual_seed(T + 7 * E + ng + k)
    scores = torch.randn((T, E), generator=gen).to(dtype)
    for renorm, bias_dtype, rsf in ((True, torch.float32, 1.0), (False, torch.bfloat16, 2.5)):
        bias = (torch.randn(E, generator=gen) * 0.1).to(bias_dtype)
        vals, ids = capi.grouped_topk(scores.cuda(), ng, tg, k, renorm, rsf, bias.cuda(),
                                      scoring)
        ref_v, ref_i = O.grouped_topk(scores.float().numpy(), ng, tg, k, renorm, rsf,
                                      bias.float().numpy(), scoring)
        ids = ids.cpu().numpy()
        x = scores.float().numpy()
        s = x if scoring == 0 else 1.0 / (1.0 + np.exp(-x))
        c = s + bias.float().numpy()[None, :]
        epg = E // ng
        exact = 0
        for r in range(T):
            assert len(set(ids[r].tolist())) == k
            np.testing.assert_allclose(c[r, ids[r]], c[r, ref_i[r]], rtol=0, atol=2e-6)
            # ids must be exact unless a deciding rank is a near-tie: the group scores around
            # the topk_group cut, or the choices around the topk cut inside the kept groups
            gs = np.sort([np.sort(c[r, g * epg:(g + 1) * epg])[-2:].sum() for g in range(ng)])
            kept = sorted({int(i) // epg for i in ref_i[r]})
            cand = np.sort(np.concatenate([c[r, g * epg:(g + 1) * epg] for g in kept]))
            if (np.all(np.abs(np.diff(gs[::-1][:tg + 1])) > 1e-6) and
                    np.all(np.abs(np.diff(cand[::-1][:k + 1])) > 1e-6)):
                assert ids[r].tolist() == ref_i[r].tolist(), f"row {r}"
                exact += 1
        chosen = np.take_along_axis(s, ids.astype(np.int64), 1)
        w = chosen * rsf
        rtol = np.full((T, 1), 1e-5)
        if renorm:
            tot = chosen.sum(1, keepdims=True)
            w = w / (1e-20 + tot)
            # the sum's order is not fixed (the reference reduces across lanes too); with
            # signed scores (scoring 0) it can cancel, which scales its rounding error by
            # sum|w| / |sum w|
            rtol = rtol + 4 * k * 2.0 ** -24 * np.abs(chosen).sum(1, keepdims=True) / np.maximum(
                np.abs(tot), 1e-30)
        err = np.abs(vals.cpu().numpy() - w)
        assert np.all(err <= 1e-6 + rtol * np.abs(w)), float((err / (1e-6 + rtol * np.abs(w))).max())
        if dtype == torch.float32:
            assert exact >= 0.9 * T


def test_grouped_topk_fallback_and_errors():
    # every input non-finite: no group scores above -inf, experts 0..k-1 with weight 1/k
    scores = torch.full((3, 16), float("inf"), device="cuda")
    vals, ids = capi.grouped_topk(scores, 4, 2, 4, True, 1.0, torch.zeros(16, device="cuda"), 1)
    assert ids.cpu().tolist() == [[0, 1, 2, 3]] * 3
    np.testing.assert_allclose(vals.cpu().numpy(), 0.25)
    # the same with 16 experts per group (group scores by cross-lane steps)
    scores = torch.full((2, 64), float("nan"), device="cuda")
    vals, ids = capi.grouped_topk(scores, 4, 2, 3, False, 1.0, torch.zeros(64, device="cuda"), 0)
    assert ids.cpu().tolist() == [[0, 1, 2]] * 2
    np.testing.assert_allclose(vals.cpu().numpy(), 1.0 / 3.0, rtol=1e-6)
    from marlin_v100_amd import _custom_ops as ops
    with pytest.raises(RuntimeError, match="num_experts should be divisible by n_group"):
        ops.grouped_topk(torch.randn((2, 10), device="cuda"), 4, 2, 2, True, 1.0,
                         torch.zeros(10, device="cuda"), 0)
    with pytest.raises(RuntimeError, match="topk_group must be <= n_group"):
        ops.grouped_topk(torch.randn((2, 16), device="cuda"), 4, 5, 2, True, 1.0,
                         torch.zeros(16, device="cuda"), 0)


def _router_case(i):
    import math
    import random

    rng = random.Random(4000 + i)
    e = max(1, int(round(2 ** rng.uniform(0, 12))))
    k = rng.randint(1, min(e, 32))
    t = max(1, int(round(2 ** rng.uniform(0, math.log2(3000)))))
    dtype = rng.choice([torch.float32, torch.float16, torch.bfloat16])
    scoring = rng.choice(["softmax", "sigmoid"])
    renorm = rng.random() < 0.5
    use_bias = rng.random() < 0.4
    return t, e, k, dtype, scoring, renorm, use_bias


ROUTER_CASES = [_router_case(i) for i in range(30)]


@pytest.mark.parametrize("i", range(len(ROUTER_CASES)))
def test_topk_random_shapes(i):
    """Seeded random shapes (1-4096 experts, top-k up to 32, 1-3000 tokens, every gating dtype,
    both scorings, with and without renormalization and a choice bias) against the oracle."""
    T, E, k, dtype, scoring, renorm, use_bias = ROUTER_CASES[i]
    print(f"case router-sweep {i}: T={T} E={E} k={k} {dtype} {scoring} renorm={renorm} "
          f"bias={use_bias}", flush=True)
    gen = torch.Generator().manual_seed(4100 + i)
    gating = (torch.randn((T, E), generator=gen) * 2).to(dtype)
    bias = (torch.randn(E, generator=gen) * 0.05) if use_bias else None
    w, ids, tei = capi.topk_gating(gating.cuda(), k, renorm,
                                   None if bias is None else bias.cuda(), scoring)
    _check(gating, k, renorm, bias, scoring, w, ids, tei)
