"""Writes the golden fixtures restated from the reference's own tests (no reference code is
imported or executed): the values below are copied from the cited test assertions.

  scalar_type_ids.json : tests/test_marlin_helpers.py:69-86 and the ScalarType table of
                         vllm/scalar_type.py:83-90 (ids as listed for the op ABI)
  moe_align_kat.json   : tests/test_marlin_moe.py:274-291 (_moe_align_block_size_reference)
  bias_perm.json       : csrc/quantization/marlin/sm70_marlin_bias.cuh:20-23
  topk_softmax_kat.json: inputs of tests/test_marlin_moe.py:248-272 (fp16 gating, fp32 bias,
                         top-2, renormalize); expected ids and weights evaluated here from the
                         closed form in float64 (softmax, selection by score + bias with ties
                         to the lower index, unbiased weights divided by their sum)
  grouped_topk_kat.json: inputs of tests/test_marlin_moe.py:313-345 (fp32 scores, sigmoid,
                         4 groups, keep 2, top-3, renormalize); expected ids and weights
                         evaluated here from the closed form in float64 (group score = sum of
                         the two largest sigmoid + bias, ties to the lower index)
"""
import json
import math
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))

FIXTURES = {
    "scalar_type_ids.json": {
        "source": "tests/test_marlin_helpers.py:69-86; vllm/scalar_type.py:25-43,83-90",
        "ids": {
            "uint4": 1125899906843648,
            "uint4b8": 1125899907892224,
            "uint8": 1125899906844672,
            "uint8b128": 1125899923621888,
            "float4_e2m1f": (2 << 0) | (1 << 8) | (1 << 16) | (1 << 49),
            "float8_e4m3fn": (4 << 0) | (3 << 8) | (1 << 16) | (1 << 49) | (2 << 50),
            "float8_e8m0fnu": (8 << 0) | (1 << 49) | (2 << 50),
        },
    },
    "moe_align_kat.json": {
        "source": "tests/test_marlin_moe.py:274-291",
        "topk_ids": [[0, 3], [1, 3], [0, 2], [1, 0]],
        "num_experts": 4,
        "block_size": 4,
        "sorted_ids": [0, 4, 7, 8, 2, 6, 8, 8, 5, 8, 8, 8, 1, 3, 8, 8],
        "expert_ids": [0, 1, 2, 3],
        "num_tokens_post_pad": 16,
    },
    "bias_perm.json": {
        "source": "csrc/quantization/marlin/sm70_marlin_bias.cuh:20-23",
        "inverse_scale_perm_single": [0, 1, 8, 9, 16, 17, 24, 25, 2, 3, 10, 11, 18, 19, 26, 27,
                                      4, 5, 12, 13, 20, 21, 28, 29, 6, 7, 14, 15, 22, 23, 30, 31],
    },
}



def _fp16(x: float) -> float:
    return struct.unpack("<e", struct.pack("<e", x))[0]


def _topk_softmax_f64(rows, bias, topk, renormalize):
    ids, weights = [], []
    for row in rows:
        m = max(row)
        ex = [math.exp(v - m) for v in row]
        p = [v / sum(ex) for v in ex]
        order = sorted(range(len(row)), key=lambda e: (-(p[e] + bias[e]), e))[:topk]
        w = [p[e] for e in order]
        if renormalize:
            s = sum(w)
            w = [v / s for v in w]
        ids.append(order)
        weights.append(w)
    return ids, weights


_GATING = [[_fp16(v) for v in r] for r in ([0.10, 0.80, -0.20, 0.30], [1.20, -0.40, 0.50, 0.10],
                                           [-0.70, 0.60, 0.20, 1.10])]
_BIAS = [struct.unpack("<f", struct.pack("<f", v))[0] for v in (0.05, -0.10, 0.20, 0.15)]
_IDS, _WEIGHTS = _topk_softmax_f64(_GATING, _BIAS, 2, True)
FIXTURES["topk_softmax_kat.json"] = {
    "source": "inputs: tests/test_marlin_moe.py:248-272; expected: float64 closed form",
    "gating_fp16_values": _GATING,
    "bias": _BIAS,
    "topk": 2,
    "renormalize": True,
    "topk_ids": _IDS,
    "topk_weights": _WEIGHTS,
    "token_expert_indices": [[t + j * 3 for j in range(2)] for t in range(3)],
}


def _f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def _grouped_topk_f64(rows, bias, n_group, topk_group, topk, renormalize, scale):
    ids, weights = [], []
    for row in rows:
        e = len(row)
        epg = e // n_group
        s = [1.0 / (1.0 + math.exp(-v)) for v in row]
        c = [s[i] + bias[i] for i in range(e)]
        gsc = [sum(sorted(c[g * epg:(g + 1) * epg], reverse=True)[:2]) for g in range(n_group)]
        kept = sorted(range(n_group), key=lambda g: (-gsc[g], g))[:topk_group]
        cand = [i for g in kept for i in range(g * epg, (g + 1) * epg)]
        sel = sorted(cand, key=lambda i: (-c[i], i))[:topk]
        w = [s[i] for i in sel]
        tot = sum(w) if renormalize else 1.0
        ids.append(sel)
        weights.append([v * scale / tot for v in w])
    return ids, weights


_GSCORES = [[_f32(v) for v in r] for r in ([0.10, 0.80, -0.40, 0.20, 1.50, 0.30, -0.10, 0.70],
                                           [0.90, -0.30, 0.40, 0.20, -0.60, 0.50, 1.10, 0.00])]
_GBIAS = [_f32(v) for v in (0.05, 0.10, -0.05, 0.00, 0.20, -0.10, 0.15, 0.05)]
_GIDS, _GWEIGHTS = _grouped_topk_f64(_GSCORES, _GBIAS, 4, 2, 3, True, 1.0)
FIXTURES["grouped_topk_kat.json"] = {
    "source": "inputs: tests/test_marlin_moe.py:313-345; expected: float64 closed form",
    "scores": _GSCORES,
    "bias": _GBIAS,
    "num_expert_group": 4,
    "topk_group": 2,
    "topk": 3,
    "renormalize": True,
    "routed_scaling_factor": 1.0,
    "scoring_func": 1,
    "topk_ids": _GIDS,
    "topk_weights": _GWEIGHTS,
}

if __name__ == "__main__":
    for name, data in FIXTURES.items():
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(data, f, indent=1)
        print("wrote", name)
