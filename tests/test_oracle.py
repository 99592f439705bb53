"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against the reference's own known-answer tests / golden
vectors where they exist (tests/golden/*.json, restated from the reference test files), and
otherwise against what the mathematics fixes (closed forms, brute force on tiny inputs,
invariants), chosen so that a plausible slip (wrong sign, wrong index, swapped nibble
order, off-by-one exponent) fails at least one check.  The planted-mistake tests at the
end perturb the oracle on the CPU and confirm the checks catch it.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# ---- scalar type ids: reference tests/test_marlin_helpers.py:69-86 ------------------------

def test_scalar_type_ids_match_reference_kat():
    g = _golden("scalar_type_ids.json")
    for name, expected in g["ids"].items():
        assert getattr(O.scalar_types, name).id == expected, name


def test_scalar_type_ids_closed_form():
    # (4 << 0) | (3 << 8) | (1 << 16) | (1 << 49) | (2 << 50) (test_marlin_helpers.py:70)
    assert O.scalar_types.float8_e4m3fn.id == (4 | 3 << 8 | 1 << 16 | 1 << 49 | 2 << 50)
    assert O.scalar_types.float4_e2m1f.id == (2 | 1 << 8 | 1 << 16 | 1 << 49)
    assert O.scalar_types.float8_e8m0fnu.id == (8 | 1 << 49 | 2 << 50)
    # integer types keep the default nan_repr = IEEE_754 (1) in bits 50..57
    assert O.scalar_types.uint4b8.id == (4 << 8 | 8 << 17 | 1 << 50)
    assert O.scalar_types.uint8b128.id == (8 << 8 | 128 << 17 | 1 << 50)


def test_product_scalar_type_matches_oracle():
    from marlin_v100_amd.scalar_type import scalar_types as P

    for name in ("uint4", "uint4b8", "uint8", "uint8b128", "float4_e2m1f", "float8_e4m3fn",
                 "float8_e8m0fnu"):
        assert getattr(P, name).id == getattr(O.scalar_types, name).id


# ---- packing -------------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [4, 8])
def test_gptq_pack_brute_force(bits):
    pack = 32 // bits
    q = torch.arange(16 * 4).reshape(16, 4) % (1 << bits)
    w = O.gptq_pack(q, bits)
    for r in range(16 // pack):
        for n in range(4):
            word = int(w[r, n]) & 0xFFFFFFFF
            for i in range(pack):
                assert (word >> (bits * i)) & ((1 << bits) - 1) == int(q[r * pack + i, n])
    assert torch.equal(O.unpack_gptq(w, bits), q.to(torch.int32))


@pytest.mark.parametrize("bits", [4, 8])
def test_awq_pack_interleave(bits):
    # tests/helpers.py:548-562: slot s of word (k, j) holds column pack*j + order[s]
    order = [0, 2, 4, 6, 1, 3, 5, 7] if bits == 4 else [0, 2, 1, 3]
    pack = 32 // bits
    q = torch.arange(4 * 16).reshape(4, 16) % (1 << bits)
    w = O.awq_pack(q, bits)
    for k in range(4):
        for j in range(16 // pack):
            word = int(w[k, j]) & 0xFFFFFFFF
            for s in range(pack):
                assert (word >> (bits * s)) & ((1 << bits) - 1) == int(q[k, pack * j + order[s]])


def test_fp4_words_low_nibble_is_even_k():
    q = torch.arange(16 * 8).reshape(16, 8) % 16
    w = O.fp4_to_gptq_words(q)
    assert w.shape == (2, 8)
    assert torch.equal(O.unpack_gptq(w, 4), q.to(torch.int32))


def test_pack_unpack_raw_nibbles_reference_vectors():
    # tests/test_marlin_helpers.py:106-119: raw = arange(16*n) % 16 survives pack/unpack
    for n in (64, 128, 192):
        raw = torch.arange(16 * n, dtype=torch.int32).reshape(16, n) % 16
        assert torch.equal(O.unpack_gptq(O.gptq_pack(raw, 4), 4), raw)


# ---- e2m1 / e8m0 / S0E5M3 ----------------------------------------------------------------

def test_fp4_table_closed_form():
    # e2m1: sign | exp(2) | mantissa(1); exp 0 is subnormal 0.5*m
    for code in range(16):
        s = -1.0 if code & 8 else 1.0
        e = (code >> 1) & 3
        m = code & 1
        v = 0.5 * m if e == 0 else (1 + 0.5 * m) * 2.0 ** (e - 1)
        assert O.FP4_VALUES[code].item() == s * v


def test_fp4_quantizer_nearest():
    vals = torch.tensor([0.24, 0.26, 1.25, 1.26, 5.0, 5.1, -2.4, 7.0])
    codes = O.quantize_to_fp4_e2m1(vals)
    assert O.FP4_VALUES[codes.long()].tolist() == [0.0, 0.5, 1.0, 1.5, 4.0, 6.0, -2.0, 6.0]


def test_s0e5m3_roundtrip_is_exact():
    # every positive e4m3 scale, both activation dtypes: decode(process(s)) == s * 2^7 * sf
    # (fp16 activations use sf = 1; every positive e4m3 value is representable)
    all_e4m3 = torch.arange(1, 127, dtype=torch.uint8).view(torch.float8_e4m3fn)
    s = all_e4m3[:124].reshape(4, 31).contiguous()
    p, sf = O.nvfp4_marlin_process_scales(s[:, :28].contiguous(), torch.float16)
    assert sf == 1.0
    assert torch.equal(O.decode_s0e5m3(p), s[:, :28].to(torch.float32) * 128.0)
    # bf16: sf lifts the smallest scale to >= 2 after *2^7; the encoding holds values up to
    # the fp16 maximum, so the check uses a 2^8-wide band of scales (as a quantizer produces)
    band = torch.arange(1, 65, dtype=torch.uint8).view(torch.float8_e4m3fn).reshape(4, 16)
    p, sf = O.nvfp4_marlin_process_scales(band.contiguous(), torch.bfloat16)
    assert sf > 1.0
    assert torch.equal(O.decode_s0e5m3(p), band.to(torch.float32) * 128.0 * sf)


def test_nvfp4_dequant_matches_direct_value():
    # tests/test_marlin_helpers.py:156-182 (atol=0): dequant of the processed metadata equals
    # dtype(e2m1 * e4m3_scale * global) computed directly
    gen = torch.Generator().manual_seed(0)
    w = torch.randn((256, 128), generator=gen) * 0.02
    q, fp8, g = O.quantize_nvfp4(w, 16)
    direct = O.FP4_VALUES[q.long()] * fp8.to(torch.float32).repeat_interleave(16, 0) * g
    for dt in (torch.float16, torch.bfloat16):
        ps, sf = O.nvfp4_marlin_process_scales(fp8, dt)
        glob = O.nvfp4_marlin_process_global_scale(g, dt) / sf
        deq = O.dequant_nvfp4(q, ps, glob, dt)
        assert torch.equal(deq, direct.to(dt))


def test_mxfp4_dequant_exact_and_close():
    # tests/test_marlin_helpers.py:185-211
    gen = torch.Generator().manual_seed(0)
    w = torch.randn((256, 128), generator=gen).half()
    q, s = O.quantize_mxfp4(w, 32)
    deq = O.dequant_mxfp4(q, s, torch.float16)
    direct = O.FP4_VALUES[q.long()] * torch.pow(2.0, s.view(torch.uint8).float() - 127).repeat_interleave(32, 0)
    assert torch.equal(deq, direct.half())
    torch.testing.assert_close(deq, w, atol=7.5e-1, rtol=7.5e-1)


# ---- integer dequant closed forms --------------------------------------------------------

def test_int_dequant_closed_forms_brute_force():
    q = torch.arange(16).reshape(16, 1).repeat(1, 2).to(torch.int32)
    s = torch.tensor([[0.03125, 0.1]], dtype=torch.float16)
    zp = torch.tensor([[0.0625, 0.7]], dtype=torch.float16)
    b8 = O.dequant_int(q, s, "u4b8", torch.float16)
    zz = O.dequant_int(q, s, "u4", torch.float16, zp)
    for i in range(16):
        for j in range(2):
            sv, zv = float(s[0, j]), float(zp[0, j])
            assert b8[i, j].item() == float(torch.tensor((i - 8) * sv).half())
            assert zz[i, j].item() == float(torch.tensor(i * sv - zv).half())


def test_zero_point_quantizer_reconstructs():
    gen = torch.Generator().manual_seed(1)
    w = torch.randn((256, 64), generator=gen) * 0.02
    q, s, z, zp = O.quantize_with_zero_point(w, 128, 4, torch.bfloat16)
    assert int(q.min()) >= 0 and int(q.max()) <= 15 and int(z.max()) <= 15
    deq = O.dequant_int(q, s, "u4", torch.bfloat16, zp).float()
    step = s.float().repeat_interleave(128, 0)
    assert ((deq - w).abs() <= step * 0.51 + 0.02 * step + 1e-4).all()


def test_bias_quantizer_reconstructs():
    gen = torch.Generator().manual_seed(2)
    w = torch.randn((256, 64), generator=gen) * 0.02
    q, s = O.quantize_with_bias(w, 128, 8, torch.float16)
    deq = O.dequant_int(q, s, "u4b8", torch.float16).float()
    step = s.float().repeat_interleave(128, 0)
    assert ((deq - w).abs() <= step * 0.51 + 1e-4).all()


def test_fp8_dequant_is_scaled_e4m3():
    fp8 = torch.arange(0, 126, dtype=torch.uint8).view(torch.float8_e4m3fn).reshape(126, 1)
    fp8 = fp8[:96].contiguous()
    s = torch.tensor([[2.0 * 256]], dtype=torch.float16)
    deq = O.dequant_fp8(fp8, s, torch.float16)
    assert torch.equal(deq, (fp8.float() * 2.0).half())


def test_bias_permutation_matches_reference_table():
    # kInverseScalePermSingle (csrc/quantization/marlin/sm70_marlin_bias.cuh:20-23)
    inv = _golden("bias_perm.json")["inverse_scale_perm_single"]
    b = torch.arange(64.0)
    p = O.marlin_permute_bias(b)
    for logical in range(64):
        assert p[(logical & ~31) + inv[logical & 31]].item() == logical


# ---- moe_align_block_size ------------------------------------------------------------------

def test_moe_align_reference_kat():
    g = _golden("moe_align_kat.json")
    s, e, n = O.moe_align_block_size(np.array(g["topk_ids"]), g["num_experts"], g["block_size"])
    assert n[0] == g["num_tokens_post_pad"]
    assert s[: n[0]].tolist() == g["sorted_ids"]
    assert e[: len(g["expert_ids"])].tolist() == g["expert_ids"]
    assert (s[n[0]:] == np.array(g["topk_ids"]).size).all()


@pytest.mark.parametrize("seed", range(5))
def test_moe_align_invariants(seed):
    rng = np.random.default_rng(seed)
    E, bs = int(rng.integers(1, 40)), int(rng.choice([4, 8, 16, 64]))
    ids = rng.integers(0, E, size=(int(rng.integers(1, 200)), int(rng.integers(1, 5))))
    s, e, n = O.moe_align_block_size(ids, E, bs)
    flat = ids.reshape(-1)
    total = n[0]
    assert total % bs == 0
    real = s[:total][s[:total] < flat.size]
    assert sorted(real.tolist()) == list(range(flat.size))  # every route exactly once
    for b in range(total // bs):
        blk = s[b * bs:(b + 1) * bs]
        valid = blk[blk < flat.size]
        assert (flat[valid] == e[b]).all()          # block holds one expert
        assert (np.diff(valid) > 0).all()            # stable (ascending) inside an expert
    assert (e[total // bs:] == -1).all()
    counts = np.bincount(flat, minlength=E)
    assert total == sum((c + bs - 1) // bs * bs for c in counts)


# ---- MoE layer reference vs the reference's per-token loop (tests/helpers.py:2039-2060) ----

def _per_token_loop(x, w1, w2, tw, ids):
    out = []
    for t in range(x.shape[0]):
        acc = torch.zeros(x.shape[1])
        row = x[t:t + 1].float()
        for r in range(ids.shape[1]):
            e = int(ids[t, r])
            g, u = (row @ w1[e].float()).chunk(2, dim=-1)
            acc += (torch.nn.functional.silu(g) * u @ w2[e].float())[0] * tw[t, r]
        out.append(acc)
    return torch.stack(out)


def test_moe_layer_ref_matches_per_token_loop():
    gen = torch.Generator().manual_seed(3)
    T, E, H, I, k = 9, 5, 32, 16, 3
    x = torch.randn((T, H), generator=gen)
    w1 = torch.randn((E, H, 2 * I), generator=gen) * 0.1
    w2 = torch.randn((E, I, H), generator=gen) * 0.1
    tw, ids = O.route_topk(torch.randn((T, E), generator=gen), k)
    torch.testing.assert_close(O.moe_layer_ref(x, w1, w2, tw, ids),
                               _per_token_loop(x, w1, w2, tw, ids), rtol=1e-5, atol=1e-5)


def test_route_topk_renormalises():
    tw, ids = O.route_topk(torch.randn((20, 64)), 8)
    torch.testing.assert_close(tw.sum(-1), torch.ones(20))
    assert ids.dtype == torch.int32 and int(ids.max()) < 64


# ---- planted mistakes: the checks above must catch a plausible slip ------------------------

def test_planted_wrong_bias_sign_is_caught(monkeypatch):
    q = torch.arange(16).reshape(16, 1).to(torch.int32)
    s = torch.tensor([[0.5]], dtype=torch.float16)
    good = O.dequant_int(q, s, "u4b8", torch.float16)
    bad = ((q.float() + 8.0) * 0.5).half()
    assert not torch.equal(good, bad)


def test_planted_swapped_nvfp4_shuffle_is_caught():
    gen = torch.Generator().manual_seed(0)
    w = torch.randn((32, 8), generator=gen) * 0.02
    q, fp8, g = O.quantize_nvfp4(w, 16)
    ps, sf = O.nvfp4_marlin_process_scales(fp8, torch.float16)
    # decoding without undoing the [0,2,1,3] shuffle must break the direct-value identity
    bits = ps.view(torch.uint8).to(torch.int16) << 7
    wrong = bits.view(torch.float16).float()
    right = O.decode_s0e5m3(ps)
    assert not torch.equal(wrong, right)


def test_planted_align_order_is_caught():
    g = _golden("moe_align_kat.json")
    s, _, n = O.moe_align_block_size(np.array(g["topk_ids"]), g["num_experts"], g["block_size"])
    reversed_within_expert = list(s[: n[0]])
    reversed_within_expert[0], reversed_within_expert[1] = reversed_within_expert[1], reversed_within_expert[0]
    assert reversed_within_expert != g["sorted_ids"]


def test_moe_sum_rounding_modes():
    # top-k 3: the reference kernel rounds after each addition in the element type
    # (moe_align_sum_kernels.cu:350-363): 1 + 2^-8 ties to 1 in bf16, twice, so the result
    # stays 1; one rounding of the fp32 sum gives 1 + 2^-7.  Top-k 8 (at::sum_out) rounds once.
    x3 = torch.tensor([[[1.0], [2.0 ** -8], [2.0 ** -8]]], dtype=torch.bfloat16)
    assert O.moe_sum(x3).item() == 1.0
    x8 = torch.cat([x3, torch.zeros((1, 5, 1), dtype=torch.bfloat16)], dim=1)
    assert O.moe_sum(x8).item() == 1.0 + 2.0 ** -7
    # top-k 2: both rules agree (the pairwise sum is exact in fp32, then one rounding)
    gen = torch.Generator().manual_seed(3)
    x2 = torch.randn((64, 2, 32), generator=gen).to(torch.bfloat16)
    assert torch.equal(O.moe_sum(x2), (x2[:, 0].float() + x2[:, 1].float()).to(torch.bfloat16))
    # top-k 1: a copy
    assert torch.equal(O.moe_sum(x2[:, :1]), x2[:, 0])


# ---- MoE router (topk_softmax / topk_sigmoid) --------------------------------------------

def test_topk_softmax_reference_kat():
    g = _golden("topk_softmax_kat.json")
    gating = np.asarray(g["gating_fp16_values"], dtype=np.float16)
    w, ids, tei = O.topk_gating(gating, g["topk"], g["renormalize"], np.asarray(g["bias"]))
    assert ids.tolist() == g["topk_ids"]
    assert tei.tolist() == g["token_expert_indices"]
    np.testing.assert_allclose(w, np.asarray(g["topk_weights"]), rtol=0, atol=1e-6)


def test_topk_closed_forms_and_tie_rule():
    ln2, ln3 = math.log(2.0), math.log(3.0)
    # probabilities [3, 1, 2, 2] / 8: the tie between experts 2 and 3 goes to 2
    x = np.array([[ln3, 0.0, ln2, ln2]], dtype=np.float32)
    w, ids, _ = O.topk_gating(x, 2)
    assert ids.tolist() == [[0, 2]]
    np.testing.assert_allclose(w, [[0.375, 0.25]], atol=1e-7)
    w, ids, _ = O.topk_gating(x, 2, renormalize=True)
    np.testing.assert_allclose(w, [[0.6, 0.4]], atol=1e-7)
    # a bias moves the choice but the weights stay the unbiased probabilities
    w, ids, _ = O.topk_gating(x, 2, True, np.array([-0.2, 0, 0, 0], np.float32))
    assert ids.tolist() == [[2, 3]]
    np.testing.assert_allclose(w, [[0.5, 0.5]], atol=1e-7)
    w, ids, _ = O.topk_gating(x, 2, False, np.array([0, 0, 0, 0.01], np.float32))
    assert ids.tolist() == [[0, 3]]
    np.testing.assert_allclose(w, [[0.375, 0.25]], atol=1e-7)
    # sigmoid(0) = 1/2, sigmoid(ln 3) = 3/4, sigmoid(-ln 3) = 1/4
    x = np.array([[0.0, ln3, -ln3]], dtype=np.float32)
    w, ids, _ = O.topk_gating(x, 2, scoring="sigmoid")
    assert ids.tolist() == [[1, 0]]
    np.testing.assert_allclose(w, [[0.75, 0.5]], atol=1e-7)
    w, ids, _ = O.topk_gating(x, 2, True, scoring="sigmoid")
    np.testing.assert_allclose(w, [[0.6, 0.4]], atol=1e-7)
    # all-equal row: experts in index order
    w, ids, tei = O.topk_gating(np.zeros((2, 5), np.float32), 5)
    assert ids.tolist() == [[0, 1, 2, 3, 4]] * 2
    assert tei.tolist() == [[0, 2, 4, 6, 8], [1, 3, 5, 7, 9]]


@pytest.mark.parametrize("seed", [0, 1])
def test_topk_invariants(seed):
    rng = np.random.default_rng(seed)
    t, e, k = 33, 96, 6
    x = rng.standard_normal((t, e)).astype(np.float32)
    bias = (0.01 * rng.standard_normal(e)).astype(np.float32)
    w, ids, _ = O.topk_gating(x, k, False, bias)
    p = torch.softmax(torch.from_numpy(x), dim=-1).numpy()  # library softmax
    choice = p + bias
    for r in range(t):
        sel = ids[r].astype(np.int64)
        assert len(set(sel.tolist())) == k
        assert np.all(np.diff(choice[r, sel]) <= 1e-7)  # non-increasing choice
        rest = np.setdiff1d(np.arange(e), sel)
        assert choice[r, rest].max() <= choice[r, sel].min() + 1e-7
    np.testing.assert_allclose(w, np.take_along_axis(p, ids.astype(np.int64), 1), rtol=1e-6)
    # renormalized weights sum to one; softmax is shift invariant
    w2, ids2, _ = O.topk_gating(x + 3.0, k, True, bias)
    assert np.array_equal(ids2, ids)
    np.testing.assert_allclose(w2.sum(axis=1), 1.0, rtol=1e-6)
    # k = E lists every expert once
    _, ids3, _ = O.topk_gating(x[:4, :16], 16)
    assert all(sorted(r) == list(range(16)) for r in ids3.tolist())


def test_planted_biased_router_weights_are_caught():
    g = _golden("topk_softmax_kat.json")
    gating = np.asarray(g["gating_fp16_values"], dtype=np.float16).astype(np.float32)
    bias = np.asarray(g["bias"], dtype=np.float32)
    _, ids, _ = O.topk_gating(gating, 2, True, bias)
    # the plausible slip: returning the biased choice score as the weight
    p = torch.softmax(torch.from_numpy(gating), dim=-1).numpy() + bias
    wrong = np.take_along_axis(p, ids.astype(np.int64), 1)
    wrong = wrong / wrong.sum(axis=1, keepdims=True)
    assert np.abs(wrong - np.asarray(g["topk_weights"])).max() > 1e-3


# ---- MoE grouped router (grouped_topk) ---------------------------------------------------

def test_grouped_topk_reference_kat():
    g = _golden("grouped_topk_kat.json")
    vals, ids = O.grouped_topk(np.asarray(g["scores"], np.float32), g["num_expert_group"],
                               g["topk_group"], g["topk"], g["renormalize"],
                               g["routed_scaling_factor"], np.asarray(g["bias"], np.float32),
                               g["scoring_func"])
    assert ids.tolist() == g["topk_ids"]
    np.testing.assert_allclose(vals, np.asarray(g["topk_weights"]), rtol=0, atol=1e-6)


def test_grouped_topk_closed_forms():
    # scoring 0 (scores as given): groups {0,1} {2,3} {4,5}; group scores 0.9, 1.1, 0.7
    x = np.array([[0.5, 0.4, 1.0, 0.1, 0.6, 0.1]], np.float32)
    z = np.zeros(6, np.float32)
    vals, ids = O.grouped_topk(x, 3, 1, 2, False, 2.5, z, 0)
    assert ids.tolist() == [[2, 3]]  # only group 1 kept, although expert 4 beats expert 3
    np.testing.assert_allclose(vals, [[2.5, 0.25]], atol=1e-7)
    vals, ids = O.grouped_topk(x, 3, 2, 3, True, 1.0, z, 0)
    assert ids.tolist() == [[2, 0, 1]]  # groups 1 and 0 kept
    np.testing.assert_allclose(vals, [[1.0 / 1.9, 0.5 / 1.9, 0.4 / 1.9]], rtol=1e-6)
    # equal group scores: the lower group wins; a -inf kept group means the 1/k fallback
    vals, ids = O.grouped_topk(np.zeros((1, 4), np.float32), 2, 1, 2, False, 1.0,
                               np.zeros(4, np.float32), 0)
    assert ids.tolist() == [[0, 1]]
    vals, ids = O.grouped_topk(np.full((1, 4), np.inf, np.float32), 2, 1, 2, True, 1.0,
                               np.zeros(4, np.float32), 1)
    assert ids.tolist() == [[0, 1]]
    np.testing.assert_allclose(vals, [[0.5, 0.5]])


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_grouped_topk_brute_force(seed):
    # tiny rows: every choice of kept groups is enumerated; the kept set must be the one with
    # the largest group scores and the experts the best choices inside it
    import itertools
    rng = np.random.default_rng(seed)
    t, e, n_group, topk_group, k = 6, 12, 4, 2, 4
    x = rng.standard_normal((t, e)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(e)).astype(np.float32)
    vals, ids = O.grouped_topk(x, n_group, topk_group, k, True, 1.5, bias, 1)
    s = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    c = s + bias
    epg = e // n_group
    for r in range(t):
        gs = [np.sort(c[r, g * epg:(g + 1) * epg])[-2:].sum() for g in range(n_group)]
        best = max(itertools.combinations(range(n_group), topk_group),
                   key=lambda sub: sum(gs[g] for g in sub))
        cand = [i for g in best for i in range(g * epg, (g + 1) * epg)]
        want = sorted(cand, key=lambda i: -c[r, i])[:k]
        assert ids[r].tolist() == want
        np.testing.assert_allclose(vals[r], 1.5 * s[r, want] / s[r, want].sum(), rtol=1e-6)


def test_planted_grouped_topk_top1_group_score_is_caught():
    # the plausible slip: scoring a group by its best expert alone.  On the closed-form row the
    # top-2 sums keep groups {1, 0} while best-expert scores would keep {1, 2}, so
    # test_grouped_topk_closed_forms fails for an oracle with that slip.
    x = np.array([0.5, 0.4, 1.0, 0.1, 0.6, 0.1], np.float32)
    top1 = sorted(range(3), key=lambda g: (-x[2 * g:2 * g + 2].max(), g))[:2]
    top2 = sorted(range(3), key=lambda g: (-np.sort(x[2 * g:2 * g + 2]).sum(), g))[:2]
    assert top2 == [1, 0] and top1 == [1, 2]
    _, ids = O.grouped_topk(x[None, :], 3, 2, 3, True, 1.0, np.zeros(6, np.float32), 0)
    assert sorted({i // 2 for i in ids[0].tolist()}) == sorted(top2)


# ---- integer zero points and act-order (upstream modes the SM70 reference rejects) --------

def test_dequant_int_zero_brute_force():
    """Every (code, zero) pair against (q - z) * s computed exactly in float64 and rounded once."""
    for dtype in (torch.float16, torch.bfloat16):
        q = torch.arange(16, dtype=torch.int32).repeat_interleave(16).reshape(256, 1)
        z = torch.arange(16, dtype=torch.int32).repeat(16).reshape(256, 1)
        s = torch.tensor([[0.0123]], dtype=dtype)
        # one group per row: expand through g_idx
        g_idx = torch.arange(256)
        zz = z.reshape(256, 1)
        ss = s.repeat(256, 1)
        got = O.dequant_int_zero(q, ss, zz, dtype, g_idx=g_idx)
        exact = ((q.double() - z.double()) * s.double()).to(dtype)
        assert torch.equal(got.view(torch.int16), exact.view(torch.int16))


def test_dequant_int_zero_agrees_with_float_zero_when_exact():
    """When z * s is representable in the dtype, the float-zero-point path (reference
    semantics, tests/helpers.py:1576-1641) gives the same single rounding."""
    gen = torch.Generator().manual_seed(1)
    k, n = 256, 64
    q = torch.randint(0, 16, (k, n), generator=gen, dtype=torch.int32)
    z = torch.randint(0, 16, (2, n), generator=gen, dtype=torch.int32)
    s = (2.0 ** -torch.randint(3, 9, (2, n), generator=gen)).to(torch.bfloat16)  # powers of two
    zp_f = (z.float() * s.float()).to(torch.bfloat16)
    assert torch.equal(zp_f.float(), z.float() * s.float())
    a = O.dequant_int_zero(q, s, z, torch.bfloat16)
    b = O.dequant_int(q, s, "u4", torch.bfloat16, zp_f)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_planted_zero_point_sign_is_caught():
    """A slip that adds the zero point instead of subtracting it fails the brute force."""
    q = torch.tensor([[3]], dtype=torch.int32)
    z = torch.tensor([[5]], dtype=torch.int32)
    s = torch.tensor([[0.5]], dtype=torch.float16)
    good = O.dequant_int_zero(q, s, z, torch.float16)
    assert good.item() == -1.0
    slipped = ((q.float() + z.float()) * s.float()).half()
    assert slipped.item() != good.item()


def test_pack_cols_closed_form():
    """Word j of row g holds codes of columns pack*j .. pack*j+pack-1, LSB first
    (quant_utils.py:66-78), brute-forced on arange codes."""
    for bits in (4, 8):
        pack = 32 // bits
        z = (torch.arange(2 * 64) % (1 << bits)).reshape(2, 64).to(torch.int32)
        w = O.pack_cols(z, bits)
        assert w.shape == (2, 64 // pack)
        for g in range(2):
            for j in range(64 // pack):
                exp = sum(int(z[g, pack * j + i]) << (bits * i) for i in range(pack))
                assert (int(w[g, j]) & 0xffffffff) == exp


def test_act_order_groups_sort_to_contiguous_groups():
    gen = torch.Generator().manual_seed(2)
    g_idx = O.act_order_groups(512, 64, gen)
    order = torch.argsort(g_idx)
    assert torch.equal(g_idx[order], (torch.arange(512) // 64).to(torch.int32))
    assert torch.equal(torch.bincount(g_idx.long()), torch.full((8,), 64))


def test_dequant_g_idx_is_a_row_permutation_of_grouped_dequant():
    """Permuting the rows of a contiguously grouped weight (and its g_idx with them) permutes
    the dequant: links dequant_int_g_idx to the pinned dequant_int."""
    gen = torch.Generator().manual_seed(3)
    k, n, gs = 256, 32, 64
    w = torch.randn((k, n), generator=gen) * 0.02
    for fmt in ("u4b8", "u4", "u8b128"):
        if fmt == "u4":
            q, s, _z, zp = O.quantize_with_zero_point(w, gs, 4, torch.float16)
        else:
            q, s = O.quantize_with_bias(w, gs, 8 if fmt == "u4b8" else 128, torch.float16)
            zp = None
        base = O.dequant_int(q, s, fmt, torch.float16, zp)
        perm = torch.randperm(k, generator=gen)
        g_idx = (torch.arange(k) // gs)[perm]
        got = O.dequant_int_g_idx(q[perm], s, fmt, torch.float16, g_idx, zp)
        assert torch.equal(got, base[perm])


def test_quantize_g_idx_reconstruction_bound():
    gen = torch.Generator().manual_seed(4)
    k, n, gs = 512, 64, 128
    g_idx = O.act_order_groups(k, gs, gen)
    w = torch.randn((k, n), generator=gen) * 0.02
    for fmt in ("u4b8", "u4", "u8b128"):
        q, s, z, zp = O.quantize_g_idx(w, g_idx, k // gs, fmt, torch.float32)
        deq = O.dequant_int_g_idx(q, s, fmt, torch.float32, g_idx, zp)
        err = (deq - w).abs()
        assert (err <= s[g_idx.long()] * 0.5 + 1e-6).all(), fmt


# ---- 8-bit-activation repack layout and the W4A8 preprocess -------------------------------

def _a8_reference_thread_walk(words: np.ndarray, size_k: int, size_n: int, bits: int):
    """The reference kernel's own walk for is_a_8bit (gptq_marlin_repack.cu:14-17, 80-107,
    224-334), restated loop by loop: a 32 x 32 tile's source words in shared-memory order,
    then each of the 4 x 32 threads assembling its word(s)."""
    pack = 32 // bits
    mask = (1 << bits) - 1
    tile_ints = 32 // pack
    tile_size = 32 * 32 // pack
    n_tiles = size_n // 32
    src = words.astype(np.int64) & 0xFFFFFFFF
    out = np.zeros(size_k * size_n // pack, dtype=np.int64)
    for kt in range(size_k // 32):
        for nt in range(n_tiles):
            sh = src[kt * tile_ints:(kt + 1) * tile_ints, nt * 32:(nt + 1) * 32].ravel()
            base = (kt * n_tiles + nt) * tile_size
            for warp in range(4):
                for th in range(32):
                    tc_col, tc_row = th // 4, (th % 4) * 4
                    cur_n = (warp // 2) * 16 + tc_col
                    b1 = [int(sh[cur_n + 32 * i + (warp % 2) * 8]) for i in range(tile_ints)]
                    vals = [0] * 8
                    for i in range(4):
                        ci, cp = (tc_row + i) // pack, (tc_row + i) % pack
                        vals[i] = (b1[ci] >> (cp * bits)) & mask
                        vals[4 + i] = (b1[ci + tile_ints // 2] >> (cp * bits)) & mask
                    if bits == 4:
                        order = [0, 4, 1, 5, 2, 6, 3, 7]
                        out[base + th * 4 + warp] = sum(vals[order[i]] << (4 * i) for i in range(8))
                    else:
                        out[base + th * 8 + warp * 2] = sum(vals[i] << (8 * i) for i in range(4))
                        out[base + th * 8 + warp * 2 + 1] = sum(vals[4 + i] << (8 * i) for i in range(4))
    return out.astype(np.uint32).view(np.int32)


@pytest.mark.parametrize("bits", [4, 8])
def test_a8_layout_matches_the_reference_thread_walk(bits):
    rng = np.random.default_rng(bits)
    k, n = 64, 96
    q = rng.integers(0, 1 << bits, size=(k, n))
    words = O.gptq_pack(torch.from_numpy(q), bits).numpy()
    got = O.a8_repack(q, bits).ravel()
    assert np.array_equal(got, _a8_reference_thread_walk(words, k, n, bits))


@pytest.mark.parametrize("bits", [4, 8])
def test_a8_layout_places_every_code_once(bits):
    k, n = 64, 64
    kk, nn = O.a8_layout_index(k, n, bits)
    flat = (kk * n + nn).ravel()
    assert np.array_equal(np.sort(flat), np.arange(k * n))


def test_a8_8bit_words_are_mma_m16n8k32_b_fragments():
    """8-bit: the two words of (thread th, n8 slice s) are the B fragment of an m16n8k32
    s8 MMA (PTX ISA, mma.m16n8k32 .s8 fragment layout): column th // 4 of the slice, rows
    (th % 4) * 4 + i (first word) and the same + 16 (second word)."""
    kk, nn = O.a8_layout_index(32, 32, 8)
    for th in range(32):
        for s in range(4):
            for h in range(2):
                w = th * 8 + 2 * s + h
                assert list(kk[w]) == [(th % 4) * 4 + 16 * h + i for i in range(4)]
                assert set(nn[w]) == {16 * (s // 2) + 8 * (s % 2) + th // 4}


def test_int4_fp8_preprocess_reference_kat():
    """tests/test_marlin_dense.py:372-388 at a smaller size: nibbles packed two per int8,
    viewed as int32; the result is v - 8 for v >= 8 and 15 - v otherwise, per nibble."""
    gen = torch.Generator().manual_seed(7)
    unpacked = torch.randint(0, 16, (128, 256), generator=gen, dtype=torch.int32)
    packed = (unpacked[:, ::2] * 16 + unpacked[:, 1::2]).to(torch.int8).view(torch.int32)
    got = O.int4_fp8_preprocess(packed.numpy())
    want = torch.where(unpacked >= 8, unpacked - 8, 15 - unpacked)
    want = (want[:, ::2] * 16 + want[:, 1::2]).to(torch.int8).view(torch.int32)
    assert np.array_equal(got, want.numpy())


def test_int4_fp8_preprocess_awq_brute_force():
    rng = np.random.default_rng(3)
    k, nw, gs = 64, 4, 32
    q = rng.integers(0, 1 << 32, size=(k, nw), dtype=np.uint64).astype(np.uint32).view(np.int32)
    z = rng.integers(0, 1 << 32, size=(k // gs, nw), dtype=np.uint64).astype(np.uint32).view(np.int32)
    got = O.int4_fp8_preprocess(q, z).view(np.uint32)
    for r in range(k):
        for c in range(nw):
            word = 0
            for i in range(8):
                v = (int(q.view(np.uint32)[r, c]) >> (4 * i)) & 15
                zz = (int(z.view(np.uint32)[r // gs, c]) >> (4 * i)) & 15
                word |= (v - zz if v >= zz else 15 - v) << (4 * i)
            assert int(got[r, c]) == word
