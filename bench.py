"""Benchmark of the Marlin hot path on one MI355X.

Headline (`value`): weight GB/s of marlin_gemm on BASELINE configs[1] -- AWQ-style uint4 +
float zero point, group 128, bf16 activations, K=5120, N=34816 -- at M=16 (decode).  One
"step" is one marlin_gemm call on that workload with all inputs resident in HBM.  Weight
copies rotate through >= 512 MiB so the 256 MB Infinity Cache cannot hold them.  Calls
shorter than 60 us are queued behind a spin kernel so they run back to back (host dispatch
would otherwise set the pace); longer ones are timed eagerly.  Both time exactly the K
calls with HIP events on the stream the kernels run on.

The same JSON line carries every other BASELINE configuration (`configs`): cfg1 u4b8 fp16,
cfg2 at M in {1,16,128,1024}, cfg3 u8b128 M=4096 (MFMA bound), cfg4 MXFP4/NVFP4 at
M in {1,64,512}, the cfg5 MoE layer (align + 2 grouped GEMMs + activation + top-k sum)
at T in {16, 2048} and its router (topk_softmax, top-8 of 256); plus `roofline` for the
headline kernel and `cpu_baseline` (the reference's CPU path: dequantize then fp32 matmul,
timed on the host cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16/fp16
ROTATE_BYTES = 512 << 20

METRIC = "marlin_gemm weight GB/s + TFLOPS vs roofline, M=1..4096; MoE layer µs"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of config keys to run")
    ap.add_argument("--warm-seconds", type=float, default=None,
                    help="wall time of untimed calls before each secondary workload (default "
                         "0.1 s; counter runs pass 0, since every dispatch is profiled)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 256 MiB device copy (counter calibration for "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only run torch.matmul (hipBLASLt) at the large-M shapes, unquantized: "
                         "the MFMA rate a vendor GEMM sustains on this part")
    return ap.parse_args()


def copy_probe(steps: int) -> int:
    """A plain copy of known size: 256 MiB read + 256 MiB written per launch."""
    import torch

    src = torch.randn(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": src.numel() * 4,
                      "copy_probe_bytes_written": dst.numel() * 4, "launches": steps}))
    return 0


def gemm_probe(steps: int) -> int:
    """torch.matmul (hipBLASLt) at the cfg3 and cfg2 M=1024 shapes with 16-bit weights: the
    MFMA rate an unquantized vendor GEMM sustains here, beside the published peak."""
    import torch

    out = {}
    for m, k, n, dt in ((4096, 8192, 8192, torch.float16), (1024, 5120, 34816, torch.bfloat16)):
        a = torch.randn(m, k, device="cuda", dtype=dt)
        b = torch.randn(k, n, device="cuda", dtype=dt)
        t = time_calls([lambda: a @ b], steps, max(3, steps // 10))
        out[f"{m}x{k}x{n}_{str(dt).replace('torch.', '')}"] = {
            "us": round(t * 1e6, 2), "TFLOPs": round(2.0 * m * k * n / t / 1e12, 1),
            "mfma_frac": round(2.0 * m * k * n / t / 1e12 / MFMA_PEAK_TFLOPS, 4)}
    print(json.dumps({"gemm_probe": out}))
    return 0


# ---------------------------------------------------------------------------------------
# synthetic quantized weights, built on the GPU (input generation, not the measured path)
# ---------------------------------------------------------------------------------------

def _pack_gptq(q, bits):
    import torch

    k, n = q.shape
    pack = 32 // bits
    qn = q.to(torch.int64).reshape(k // pack, pack, n)
    out = torch.zeros((k // pack, n), dtype=torch.int64, device=q.device)
    for i in range(pack):
        out |= qn[:, i, :] << (bits * i)
    out = torch.where(out >= 2 ** 31, out - 2 ** 32, out)
    return out.to(torch.int32)


FP4_GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def make_weights(fmt, k, n, dtype, gen, experts=None):
    """RTN-quantize W ~ N(0, 0.02) [K, N] in `fmt`; returns dict of kernel operands."""
    import torch

    from marlin_v100_amd import ops
    from marlin_v100_amd.marlin_utils import (nvfp4_marlin_process_global_scale,
                                              nvfp4_marlin_process_scales)

    w = (torch.randn((k, n), generator=gen, device="cuda") * 0.02)
    out = {}
    if fmt == "u4b8":
        g = k // 128
        r = w.reshape(g, 128, n)
        s = (r.abs().amax(1) / 7).clamp_min(1e-6).to(dtype)
        q = (torch.round(r / s.float().unsqueeze(1)).clamp(-8, 7) + 8).reshape(k, n)
        out.update(words=_pack_gptq(q, 4), scales=s, bits=4)
    elif fmt == "u4":
        g = k // 128
        r = w.reshape(g, 128, n)
        mn, mx = r.amin(1), r.amax(1)
        s32 = ((mx - mn) / 15).clamp_min(1e-6)
        z = torch.round(-mn / s32).clamp(0, 15)
        q = torch.round(r / s32.unsqueeze(1) + z.unsqueeze(1)).clamp(0, 15).reshape(k, n)
        s = s32.to(dtype)
        out.update(words=_pack_gptq(q, 4), scales=s, zeros=(z * s.float()).to(dtype), bits=4)
    elif fmt == "u8b128":
        s = (w.abs().amax(0, keepdim=True) / 127).clamp_min(1e-6).to(dtype)
        q = torch.round(w / s.float()).clamp(-128, 127) + 128
        out.update(words=_pack_gptq(q, 8), scales=s, bits=8)
    elif fmt in ("mxfp4", "nvfp4"):
        gs = 32 if fmt == "mxfp4" else 16
        r = w.reshape(k // gs, gs, n)
        grid = torch.tensor(FP4_GRID, device="cuda")
        amax = r.abs().amax(1)
        if fmt == "mxfp4":
            e = torch.ceil(torch.log2((amax / 6).clamp_min(2.0 ** -127)))
            sc = torch.pow(2.0, e).to(torch.float8_e8m0fnu)
            eff = sc.float()
        else:
            sc32 = (amax / 6).clamp_min(1e-6)
            glob = (sc32.max() / 448).reshape(1)
            sc = (sc32 / glob).to(torch.float8_e4m3fn)
            eff = sc.float() * glob
        x = r / eff.unsqueeze(1)
        q = (x.unsqueeze(-1) - grid).abs().argmin(-1).reshape(k, n)
        words = _pack_gptq(q, 4)
        if fmt == "mxfp4":
            out.update(words=words, scales=sc.contiguous(), bits=4)
        else:
            ps, sf = nvfp4_marlin_process_scales(sc, a_dtype=dtype)
            gsc = (nvfp4_marlin_process_global_scale(glob, dtype) / sf).float()
            out.update(words=words, scales=ps, global_scale=gsc, bits=4)
    else:
        raise ValueError(fmt)
    out["qweight"] = ops.gptq_marlin_repack(out.pop("words"), torch.empty(0, dtype=torch.int32,
                                                                           device="cuda"),
                                            k, n, out["bits"])
    return out


def meta_bytes(wt):
    b = wt["qweight"].numel() * 4
    for key in ("scales", "zeros", "global_scale"):
        if wt.get(key) is not None:
            b += wt[key].numel() * wt[key].element_size()
    return b


# ---------------------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------------------

# untimed calls before every measurement run for at least this long: after an idle spell the
# GPU's clocks take ~20-30 ms of sustained work to come back up (the cfg5 T = 2048 MoE layer
# measured 1094, 1039, 980, 929 ... 904 us over its first ten 5-call rounds, and again after
# a 2 s pause), which three warm-up calls of a 1 ms layer do not cover.  The HBM-bound
# headline decode is insensitive to it (22.2-22.4 us either way).
WARM_SECONDS = 0.1


def warm_up(fn_list, warmup, seconds=None):
    """At least `warmup` calls, and calls until `seconds` (default WARM_SECONDS) of wall time
    have passed."""
    import torch

    if seconds is None:
        seconds = WARM_SECONDS

    n = len(fn_list)
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < seconds:
        fn_list[i % n]()
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_calls(fn_list, steps, warmup, warm_seconds=None):
    """Average per-call device time of rotating calls, HIP events on the current stream."""
    import torch

    n = len(fn_list)
    warm_up(fn_list, warmup, warm_seconds)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn_list[i % n]()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def time_queued(fn_list, steps, warmup, warm_seconds=None):
    """Average per-call device time with the host out of the critical path: after an eager
    warm-up, a bounded spin kernel (torch.cuda._sleep) is queued ahead of the start event, so
    the GPU is busy while the host enqueues the K timed calls; they then run back to back and
    the HIP events (on the stream the kernels run on) time the kernels, not the host's
    dispatch rate.  No graph: on this stack a captured graph adds a per-node gap."""
    import torch

    n = len(fn_list)
    warm_up(fn_list, warmup, warm_seconds)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(SPIN_CYCLES)
    start.record()
    for i in range(steps):
        fn_list[i % n]()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


# spin ahead of the timed calls (tens of ms at GPU clock rates; longer than enqueueing them)
SPIN_CYCLES = 50_000_000

# calls shorter than this are timed with the host queued ahead (host dispatch would
# otherwise set the pace)
QUEUED_BELOW_US = 60.0


def dense_case(key, fmt, m, k, n, dtype, steps, warmup, seed, warm_seconds=None):
    import torch

    from marlin_v100_amd import ops
    from marlin_v100_amd.scalar_type import scalar_types

    qtype = {"u4b8": scalar_types.uint4b8, "u4": scalar_types.uint4,
             "u8b128": scalar_types.uint8b128, "mxfp4": scalar_types.float4_e2m1f,
             "nvfp4": scalar_types.float4_e2m1f}[fmt]
    gen = torch.Generator(device="cuda").manual_seed(seed)
    first = make_weights(fmt, k, n, dtype, gen)
    wbytes = meta_bytes(first)
    # distinct weight copies rotated through >= 512 MiB (twice the 256 MB Infinity Cache), so
    # every call streams its weights from HBM
    copies = max(1, -(-ROTATE_BYTES // wbytes))
    weights = [first] + [make_weights(fmt, k, n, dtype, gen) for _ in range(copies - 1)]
    a = torch.randn((m, k), generator=gen, device="cuda").to(dtype)
    c = torch.empty((m, n), device="cuda", dtype=dtype)
    ws = torch.empty(0, dtype=torch.int32, device="cuda")

    def call(wt):
        return lambda: ops.marlin_gemm(a, c, wt["qweight"], None, wt["scales"], None,
                                       wt.get("global_scale"), wt.get("zeros"), None, None, ws,
                                       qtype, m, n, k, True, False, False,
                                       wt.get("zeros") is not None)

    fns = [call(wt) for wt in weights]
    t = time_calls(fns, steps, warmup, warm_seconds)
    timing = "eager"
    if t * 1e6 < QUEUED_BELOW_US:
        t = time_queued(fns, steps, warmup, warm_seconds)
        timing = "queued"
    alg_bytes = wbytes + a.numel() * 2 + c.numel() * 2
    flops = 2.0 * m * n * k
    gbs = alg_bytes / t / 1e9
    tflops = flops / t / 1e12
    bound = "hbm" if alg_bytes / (HBM_PEAK_GBS * 1e9) >= flops / (MFMA_PEAK_TFLOPS * 1e12) else "mfma"
    return {
        "key": key, "fmt": fmt, "dtype": str(dtype).replace("torch.", ""), "M": m, "K": k, "N": n,
        "us": round(t * 1e6, 2), "weight_GBs": round(wbytes / t / 1e9, 1),
        "alg_GBs": round(gbs, 1), "TFLOPs": round(tflops, 2), "bound": bound,
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "mfma_frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
        "alg_bytes": alg_bytes, "weight_bytes": wbytes, "flops": flops, "rotated_copies": copies,
        "rotated_bytes": copies * wbytes, "timing": timing,
    }


def moe_case(key, tokens, steps, warmup, seed):
    """cfg5: E=256, top-8, H=3072, I=1536, uint4 + float zp g128, bf16, block 64."""
    import torch

    from marlin_v100_amd.fused_marlin_moe import fused_marlin_moe
    from marlin_v100_amd.scalar_type import scalar_types

    E, topk, H, I, bs = 256, 8, 3072, 1536, 64
    dtype = torch.bfloat16
    gen = torch.Generator(device="cuda").manual_seed(seed)
    w13 = [make_weights("u4", H, 2 * I, dtype, gen) for _ in range(E)]
    w2 = [make_weights("u4", I, H, dtype, gen) for _ in range(E)]
    q13 = torch.stack([w["qweight"] for w in w13]); s13 = torch.stack([w["scales"] for w in w13])
    z13 = torch.stack([w["zeros"] for w in w13])
    q2 = torch.stack([w["qweight"] for w in w2]); s2 = torch.stack([w["scales"] for w in w2])
    z2 = torch.stack([w["zeros"] for w in w2])
    del w13, w2
    x = torch.randn((tokens, H), generator=gen, device="cuda").to(dtype)
    logits = torch.randn((tokens, E), generator=gen, device="cuda")
    p = torch.softmax(logits, -1)
    tw, ids = torch.topk(p, topk, -1)
    tw = (tw / tw.sum(-1, keepdim=True)).float().contiguous()
    ids = ids.to(torch.int32).contiguous()
    qid = scalar_types.uint4.id

    def fn():
        return fused_marlin_moe(x, q13, q2, None, None, s13, s2, tw, ids, qid, w1_zeros=z13,
                                w2_zeros=z2, is_w1_zp_float=True, is_w2_zp_float=True,
                                block_size_m=bs)

    t = time_calls([fn], steps, warmup)
    touched = int(torch.unique(ids).numel())
    per_expert = (q13[0].numel() + q2[0].numel()) * 4 + (s13[0].numel() + z13[0].numel()
                                                         + s2[0].numel() + z2[0].numel()) * 2
    alg_bytes = touched * per_expert + 2 * tokens * H * 2
    flops = 2.0 * tokens * topk * (H * 2 * I + I * H)
    roof = max(alg_bytes / (HBM_PEAK_GBS * 1e9), flops / (MFMA_PEAK_TFLOPS * 1e12))
    return {"key": key, "T": tokens, "E": E, "topk": topk, "H": H, "I": I, "block": bs,
            "layer_us": round(t * 1e6, 2), "touched_experts": touched, "alg_bytes": alg_bytes,
            "flops": flops, "roofline_us": round(roof * 1e6, 2),
            "vs_roofline": round(t / roof, 3)}


def router_case(key, tokens, steps, warmup, seed, grouped=False):
    """cfg5 router: topk_softmax over fp32 logits [T, 256], top-8, renormalized.  grouped:
    grouped_topk at the DeepSeek-V3 routing shape (256 experts in 8 groups, keep 4, top-8,
    sigmoid + fp32 bias, renormalized, scale 2.5) on the same logits."""
    import torch

    from marlin_v100_amd import _custom_ops as ops

    E, topk = 256, 8
    gen = torch.Generator(device="cuda").manual_seed(seed)
    logits = torch.randn((tokens, E), generator=gen, device="cuda")
    bias = torch.randn(E, generator=gen, device="cuda") * 0.1
    w = torch.empty((tokens, topk), dtype=torch.float32, device="cuda")
    ids = torch.empty((tokens, topk), dtype=torch.int32, device="cuda")
    tei = torch.empty((tokens, topk), dtype=torch.int32, device="cuda")

    def fn():
        if grouped:
            ops.grouped_topk(logits, 8, 4, topk, True, 2.5, bias, 1)
        else:
            ops.topk_softmax(w, ids, tei, logits, True, None)

    # eager calls are bound by host dispatch (torch op -> C ABI -> launch); the device rate
    # comes from the same calls queued behind a spin kernel
    t_eager = time_calls([fn], steps, warmup)
    t = time_queued([fn], steps, warmup)
    alg_bytes = tokens * E * 4 + tokens * topk * 12
    return {"key": key, "T": tokens, "E": E, "topk": topk, "us": round(t * 1e6, 2),
            "us_eager_dispatch": round(t_eager * 1e6, 2), "alg_bytes": alg_bytes,
            "alg_GBs": round(alg_bytes / t / 1e9, 1),
            "hbm_frac": round(alg_bytes / t / 1e9 / HBM_PEAK_GBS, 4)}


# ---------------------------------------------------------------------------------------
# CPU reference path (bounded sample), timed on the host cores
# ---------------------------------------------------------------------------------------

def cpu_threads() -> int:
    """Host threads for the CPU baseline: the CPUs this process may run on, capped by
    OMP_NUM_THREADS when the job sets it (the GPU box grants each job a CPU share and sets
    OMP_NUM_THREADS to it)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(m, k, n):
    """The reference's CPU path on the headline workload: dequantize (the oracle's
    restatement of the reference dequant) then fp32 torch.matmul (tests/helpers.py:1749-1760),
    each timed separately, median of 5 after one warm-up, on a bounded column slice."""
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle as O

    cores = cpu_threads()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(1001)
    # bounded sample: the full K, a 4096-column slice of N (weights dominate the work)
    ns = min(n, 4096)
    w = torch.randn((k, ns), generator=gen) * 0.02
    q, s, _z, zp = O.quantize_with_zero_point(w, 128, 4, torch.bfloat16)
    a = torch.randn((m, k), generator=gen).bfloat16()

    def dequant():
        return O.dequant_int(q, s, "u4", torch.bfloat16, zp)

    deq = dequant()
    O.gemm_ref(a, deq)
    t_deq, t_mm = [], []
    t_end = time.time() + 20.0
    while len(t_deq) < 5 or (time.time() < t_end and len(t_deq) < 25):
        t0 = time.perf_counter()
        deq = dequant()
        t1 = time.perf_counter()
        O.gemm_ref(a, deq)
        t2 = time.perf_counter()
        t_deq.append(t1 - t0)
        t_mm.append(t2 - t1)
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    td, tm = med(t_deq), med(t_mm)
    t = td + tm
    wbytes = k * ns // 2 + 2 * (k // 128) * ns * 2
    return {"value": round(wbytes / t / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"oracle dequant (uint4+zp g128 -> bf16) + fp32 torch.matmul, "
                      f"M={m} K={k} N={ns} (column slice of N={n}), median of {len(t_deq)} runs "
                      f"after one warm-up, {cores} threads",
            "ms_per_call": round(t * 1e3, 2), "dequant_ms": round(td * 1e3, 2),
            "matmul_ms": round(tm * 1e3, 2)}


def main() -> int:
    global WARM_SECONDS
    args = parse()
    if args.warm_seconds is not None:
        WARM_SECONDS = args.warm_seconds
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(the path's multi-GPU sharding is designed, not run)"}))
        return 2
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    if args.copy_probe:
        return copy_probe(args.steps)
    if args.gemm_probe:
        return gemm_probe(args.steps)
    from marlin_v100_amd import ops  # noqa: F401  (loads the native libraries; no fallback)

    only = set(filter(None, args.only.split(",")))
    bf, hf = torch.bfloat16, torch.float16
    # (the headline keeps exactly the driver's W warm-up calls; it does not depend on how warm
    # the GPU is, see WARM_SECONDS)
    head = dense_case("cfg2_m16", "u4", 16, 5120, 34816, bf, args.steps, args.warmup, 1002,
                      warm_seconds=0.0)

    plan = [
        ("cfg1_m16", "u4b8", 16, 4096, 4096, hf, 1001),
        ("cfg2_m1", "u4", 1, 5120, 34816, bf, 1002),
        ("cfg2_m128", "u4", 128, 5120, 34816, bf, 1002),
        ("cfg2_m1024", "u4", 1024, 5120, 34816, bf, 1002),
        ("cfg3_m4096", "u8b128", 4096, 8192, 8192, hf, 1003),
        ("cfg4_mxfp4_m1", "mxfp4", 1, 3072, 12288, bf, 1004),
        ("cfg4_mxfp4_m64", "mxfp4", 64, 3072, 12288, bf, 1004),
        ("cfg4_mxfp4_m512", "mxfp4", 512, 3072, 12288, bf, 1004),
        ("cfg4_nvfp4_m1", "nvfp4", 1, 3072, 12288, bf, 1004),
        ("cfg4_nvfp4_m64", "nvfp4", 64, 3072, 12288, bf, 1004),
        ("cfg4_nvfp4_m512", "nvfp4", 512, 3072, 12288, bf, 1004),
    ]
    configs = {"cfg2_m16": head}
    if not args.quick:
        for key, fmt, m, k, n, dt, seed in plan:
            if only and key not in only:
                continue
            steps = max(20, args.steps // (4 if m >= 1024 else 1))
            configs[key] = dense_case(key, fmt, m, k, n, dt, steps, args.warmup, seed)
            print(f"# {key}: {configs[key]['us']} us", file=sys.stderr, flush=True)
        for key, t in (("cfg5_moe_t16", 16), ("cfg5_moe_t2048", 2048)):
            if only and key not in only:
                continue
            configs[key] = moe_case(key, t, max(10, args.steps // 10), max(3, args.warmup // 4), 1005)
            print(f"# {key}: {configs[key]['layer_us']} us", file=sys.stderr, flush=True)
        for key, t, grouped in (("cfg5_router_t16", 16, False), ("cfg5_router_t2048", 2048, False),
                                ("router_grouped_topk_t2048", 2048, True)):
            if only and key not in only:
                continue
            configs[key] = router_case(key, t, args.steps, args.warmup, 1005, grouped)
            print(f"# {key}: {configs[key]['us']} us", file=sys.stderr, flush=True)

    t = head["us"] / 1e6
    # HBM traffic per launch of the headline kernel, from the rocprofv3 FETCH_SIZE /
    # WRITE_SIZE runs (copy-kernel calibrated) recorded in profiles/ for this workload.
    traffic = None
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                         "traffic_cfg2_m16.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("traffic_bytes")
    line = {
        "metric": METRIC,
        "value": head["weight_GBs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (W ~ N(0,0.02) RTN-quantized on device, A ~ N(0,1))",
        "config": {"workload": "cfg2: marlin_gemm uint4+zp g128 bf16, M=16 K=5120 N=34816 "
                               "(AWQ-style, decode)", "M": 16, "K": 5120, "N": 34816,
                   "group_size": 128, "b_type": "uint4", "act": "bf16",
                   "cold_cache_rotation_copies": head["rotated_copies"]},
        "roofline": {"bound": "hbm", "achieved": head["alg_GBs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["alg_GBs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": "mmi::marlin_decode_kernel<FMT_U4, BF16, NT=4, DEPTH=3, "
                               "WPB=4, KSPLIT, GSM_BIG, dense, OCC=3>",
                     "algorithmic_bytes_per_launch": head["alg_bytes"]},
        "configs": configs,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(16, 5120, 34816)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
