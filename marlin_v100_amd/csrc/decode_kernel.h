// decode_kernel.h -- weight-streaming GEMM for M <= 16 (decode), gfx950.
//
// At M <= 16 the GEMM is bound by streaming the packed weights from HBM, and the kernel's
// job is to keep enough weight bytes in flight on every CU without ever making waves wait
// on each other inside the K loop:
//   * each wave owns NT n16 tiles (16*NT columns) and a range of K steps (128 deep).  The
//     WPB waves of a workgroup either split the K range of one column group (KSPLIT: their
//     partial sums are added through LDS once at the end, no global atomics) or own
//     adjacent column groups over the same K range;
//   * per step each lane loads one dwordx4 of the chunk-major weight layout
//     (device_common.h) per tile, the step's scale metadata and its share of the step's
//     activations into a register ring of DEPTH slots, so DEPTH-1 steps of weights are in
//     flight while one is multiplied.  (A ring in LDS, filled by global_load_lds_dwordx4,
//     would save the registers, but the compiler's wait-count insertion does not tell the
//     slots of such a ring apart and waits for every pending copy before each LDS read.);
//   * dense blocks load the activations four whole rows per instruction and pass them
//     through a per-wave LDS tile into the MFMA operand layout (half the L1 cache-line
//     requests of loading the operand layout directly); MoE blocks gather rows by route;
//   * slots are compile-time indices (static_for), the loop body is branch-free, loads are
//     issued in one fixed order on every path into the loop, so the compiler's vmcnt
//     bookkeeping waits only for the step it consumes;
//   * OCC = 3 instances fit three waves per SIMD (activations then run one step behind the
//     weights, and the tiles are multiplied two at a time), so a launch of up to three
//     workgroups per CU is resident in one round; the few-routes MoE blocks use the same
//     register-lean order at OCC = 2 (two one-wave workgroups per SIMD);
//   * integer and fp8 weights use the integer-operand path (device_common.h): the MFMA B
//     operand is the code itself and the scale / zero point is applied per group to the
//     fp32 partial sums;
//   * K split across workgroups (when the grid needs it): the split blocks come first in
//     the grid, add fp32 partial sums into a workspace with device-scope atomics, and the
//     last arriver of a column group finishes it (arrival counters, as in gemm_kernel.h);
//   * GATED (MoE stage 1 with the SiLU-gated activation fused, one wave per workgroup):
//     a wave's four tiles are two gate tiles and the two up tiles N/2 columns later, so
//     each lane holds both factors of its outputs and stores silu(gate) * up, rounded as
//     stage 1's store followed by silu_and_mul would round it.
#pragma once

#include <type_traits>

#include "gemm_kernel.h"

namespace mmi {

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N-1>), fully unrolled.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// OCC: waves per SIMD the register allocation must allow (1 = compiler's choice).  At
// OCC >= 2 the activation slices, which hit in L2, are loaded one step later than the weights
// (ALEAD < DEPTH - 1), so fewer ring slots are live at once, and grouped integer-operand
// tiles are multiplied and scaled two at a time.
template <int FMT, class AT, int NT, int DEPTH, int WPB, bool KSPLIT, int GSM, bool MOE, int OCC,
          bool GATED = false>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(OCC, 8)))
void marlin_decode_kernel(const GemmParams p) {
  static_assert(!MOE || KSPLIT, "MoE blocks use the K-split workgroup layout");
  static_assert(!GATED || (MOE && NT == 4 && WPB == 1), "gated: one-wave MoE blocks, 4 tiles");
  constexpr int BITS = fmt_bits(FMT);
  constexpr int NL = (BITS == 4) ? 1 : 2;  // 1 KiB chunks per tile per 128-deep step
  constexpr int RAWB = (GSM == GSM_SMALL) ? 4 : 1;
  static_assert(DEPTH >= 2 && DEPTH <= 4, "ring depth");
  constexpr int ALEAD = (OCC >= 2 && DEPTH >= 3) ? DEPTH - 2 : DEPTH - 1;

  const int lane = threadIdx.x & 63;
  // (readfirstlane: the wave index is uniform, so the K range, the loop counter and the
  // per-step addresses derived from it live in SGPRs)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lg = lane >> 4;
  const int ln = lane & 15;
  const uint32_t vz = opaque_zero(p.zero);

  // grid: (split fastest, then block); n_blk indexes column groups.  MoE (reference
  // sm70_marlin_gemm.cuh:3591-3686): blocks are (moe block, column group), column group
  // fastest; the moe block's rows (<= 64) are read with one load per lane, and only its
  // 16-row parts that hold routes are multiplied, one after the other.  Rows are gathered by
  // route id / top_k and scattered to route id.
  // Blocks [0, nleft) split K `splits` ways over the column groups from main_blocks on; they
  // come first so that their waves are the oldest on each CU (issue priority goes to older
  // waves) and their short K ranges and atomics finish under the main blocks' streaming.
  // Blocks from nleft on take one whole column group each.
  const int nleft = (int)gridDim.x - p.main_blocks;
  int split = 0;
  int blk = (int)blockIdx.x - nleft;
  int nsplit = 1;
  if ((int)blockIdx.x < nleft) {
    split = blockIdx.x % p.splits;
    blk = p.main_blocks + blockIdx.x / p.splits;
    nsplit = p.splits;
  }
  int n_blk = KSPLIT ? blk : blk * WPB + wave;
  int expert = 0;
  int route = -1;      // MoE: route index of block row `lane`
  float route_w = 1.0f;  // MoE: its router weight (1 without mul_topk), read once here
  uint64_t live = 1;   // MoE: rows holding routes
  int nparts = 1;
  if constexpr (MOE) {
    n_blk = blk % p.num_n_blocks;
    const int m_blk = blk / p.num_n_blocks;
    const int padded = p.num_post_pad[0];
    if (m_blk * p.moe_bs >= padded || m_blk >= p.expert_ids_numel) return;
    expert = p.expert_ids[m_blk];
    if (expert < 0) return;
    const int si = m_blk * p.moe_bs + lane;
    if (lane < p.moe_bs && si < p.sorted_numel && si < padded) {
      const int id = p.sorted_ids[si];
      if (id >= 0 && id < p.valid_ids) route = id;
    }
    if (p.mul_topk && route >= 0) route_w = p.topk_w[route];
    live = __ballot(route >= 0);
    nparts = (p.moe_bs + 15) >> 4;
  }
  // n16 tile of the wave's tile t (GATED: tiles 0-1 are gate columns 32 n_blk.., tiles 2-3
  // the up columns N/2 later)
  const int tn0 = GATED ? 2 * n_blk : n_blk * NT;
  const int up_skip = GATED ? (p.N >> 5) - 2 : 0;
  auto col_tile = [&](int t) __attribute__((always_inline)) {
    return tn0 + t + ((GATED && t >= 2) ? up_skip : 0);
  };

  for (int part = 0; part < nparts; ++part) {
  // (every wave of the workgroup sees the same rows, so the part loop is uniform)
  if (MOE && ((live >> (16 * part)) & 0xffffull) == 0) continue;
  const int row_id = MOE ? __shfl(route, part * 16 + ln) : -1;

  const uint16_t* a = reinterpret_cast<const uint16_t*>(p.a);
  const int64_t a_r = MOE ? (row_id >= 0 ? row_id / p.top_k : 0) : min(ln, p.M - 1);
  const uint16_t* a_row = a + a_r * p.a_stride + 8 * lg;
  // Dense blocks load each step's activations line by line (lane l of load b takes 16
  // bytes of row 4b + l/16 at k offset 8*(l%16), so a load covers four whole rows) and pass
  // them through a per-wave LDS tile into the MFMA operand layout, instead of 16 rows x 64
  // bytes per load: half the L1 cache-line requests for the same bytes.
  constexpr bool ATX = !MOE;
  int a_off[4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
    a_off[b] = min(4 * b + (lane >> 4), p.M - 1) * (int)p.a_stride + 8 * (lane & 15);

  const int64_t chunk_stride = (int64_t)(p.N >> 4) * 256;
  const uint32_t* bbase = p.b + (int64_t)expert * p.b_expert_stride;
  const uint32_t* bptr = bbase + (int64_t)tn0 * 256 + lane * 4;
  const int64_t meta_base = (int64_t)expert * p.meta_expert_stride;

  const int total_full = p.K / 128;
  const int k_tail = p.K - total_full * 128;
  int s_begin = split * p.steps_per_split;
  int s_end = nsplit == 1 ? total_full : min(total_full, s_begin + p.steps_per_split);
  bool do_tail = (k_tail != 0) && (split == nsplit - 1);
  if constexpr (KSPLIT) {
    const int per_wave = (max(s_end - s_begin, 0) + WPB - 1) / WPB;
    s_begin += wave * per_wave;
    s_end = min(s_end, s_begin + per_wave);
    do_tail = do_tail && wave == WPB - 1;
  }

  f32x4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Integer-operand path (scale after the MFMA) for the integer and fp8 formats with one
  // scale per column or per >= 128-deep group; dequantize-then-multiply otherwise.
  using IO = IntOperand<FMT, AT>;
  constexpr bool INT_B = IO::kEnabled && GSM != GSM_SMALL;
  constexpr bool ROWSUM = INT_B && IO::kNeedRowSum;
  f32x4_t rsum = f32x4_t{0.f, 0.f, 0.f, 0.f};  // channelwise: row sums over all of K

  Meta meta_ch[NT];
  if constexpr (GSM == GSM_CHANNEL && !INT_B) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
      meta_ch[t] = make_meta<FMT, AT>(load_meta_raw<FMT, AT>(p, meta_base, 0, col_tile(t) * 16 + ln));
  }

  u32x4_t ra[DEPTH][4];       // activations: 4 k32 blocks per step
  u32x4_t rb[DEPTH][NT][NL];  // weights
  MetaRaw rm[DEPTH][NT][RAWB];

  auto load_meta = [&](int k0, MetaRaw (&mv)[NT][RAWB]) __attribute__((always_inline)) {
    if constexpr (GSM == GSM_BIG) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        mv[t][0] = load_meta_raw<FMT, AT>(p, meta_base, k0 >> p.group_shift, col_tile(t) * 16 + ln);
    } else if constexpr (GSM == GSM_SMALL) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          mv[t][b] = load_meta_raw<FMT, AT>(p, meta_base, (k0 + 32 * b + 8 * lg) >> p.group_shift,
                                            col_tile(t) * 16 + ln);
    }
  };

  // Issue the weights and metadata of step s into ring slot dc.
  // (issue_order: the prologue and the loop issue weights, metadata and activations in the
  // same fixed order, so the wait counts the compiler derives for the loop header hold on
  // both paths into it and keep DEPTH-1 steps in flight.)
  auto load_b = [&](int s, auto dc) __attribute__((always_inline)) {
    constexpr int d = decltype(dc)::value;
    issue_order();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t* tp = bptr + (col_tile(t) - tn0) * 256 + (int64_t)s * NL * chunk_stride;
#pragma unroll
      for (int c = 0; c < NL; ++c)
        rb[d][t][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(tp + c * chunk_stride));
    }
    issue_order();
    load_meta(s * 128, rm[d]);
    issue_order();
  };
  // Issue the activation slices of step s into ring slot dc.
  auto load_a = [&](int s, auto dc) __attribute__((always_inline)) {
    constexpr int d = decltype(dc)::value;
    const int k0 = s * 128;
    issue_order();
#pragma unroll
    for (int b = 0; b < 4; ++b)
      ra[d][b] = ATX ? *reinterpret_cast<const u32x4_t*>(a + a_off[b] + k0)
                     : *reinterpret_cast<const u32x4_t*>(a_row + k0 + 32 * b);
    issue_order();
  };

  auto b_words = [&](const u32x4_t (&bv)[NT][NL], int t, int b, uint32_t& w0, uint32_t& w1) __attribute__((always_inline)) {
    if constexpr (BITS == 4) {
      w0 = bv[t][0][b];
      w1 = 0;
    } else {
      w0 = bv[t][b >> 1][(b & 1) * 2];
      w1 = bv[t][b >> 1][(b & 1) * 2 + 1];
    }
  };

  auto compute_regs = [&](const u32x4_t (&av)[4], const u32x4_t (&bv)[NT][NL],
                          const MetaRaw (&mv)[NT][RAWB], int nblocks, auto permuted)
                          __attribute__((always_inline)) {
    constexpr bool PERMUTED = decltype(permuted)::value;
    if constexpr (INT_B && GSM != GSM_CHANNEL && OCC >= 2) {
      // grouped, register-lean order: the step's row sums first, then the tiles two at a
      // time, each pair scaled into acc as soon as its four k32 blocks are multiplied
      f32x4_t r = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const u32x4_t ones = u32x4_t{IO::kOnes, IO::kOnes, IO::kOnes, IO::kOnes};
      if constexpr (ROWSUM) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (b < nblocks) r = mfma16(av[b], ones, r, AT{});
      }
      constexpr int TP = NT >= 2 ? 2 : 1;
#pragma unroll
      for (int t0 = 0; t0 < NT; t0 += TP) {
        f32x4_t d[TP];
#pragma unroll
        for (int u = 0; u < TP; ++u) d[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (b < nblocks) {
            const u32x4_t ap = (BITS == 4 && !PERMUTED) ? a_perm_u4(av[b]) : av[b];
#pragma unroll
            for (int u = 0; u < TP; ++u) {
              uint32_t w0, w1;
              b_words(bv, t0 + u, b, w0, w1);
              d[u] = mfma16(ap, int_operand<FMT, AT>(w0, w1, vz), d[u], AT{});
            }
          }
        }
#pragma unroll
        for (int u = 0; u < TP; ++u) {
          const IMeta m = make_imeta<FMT, AT>(mv[t0 + u][0]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = __builtin_fmaf(m.S, d[u][i], acc[t0 + u][i]);
            if constexpr (ROWSUM) v = __builtin_fmaf(-m.C, r[i], v);
            acc[t0 + u][i] = v;
          }
        }
      }
    } else if constexpr (INT_B) {
      // channelwise: accumulate D and R over all of K; grouped: per step, then scale
      f32x4_t d[NT];
      f32x4_t r;
#pragma unroll
      for (int t = 0; t < NT; ++t) d[t] = GSM == GSM_CHANNEL ? acc[t] : f32x4_t{0.f, 0.f, 0.f, 0.f};
      r = GSM == GSM_CHANNEL ? rsum : f32x4_t{0.f, 0.f, 0.f, 0.f};
      const u32x4_t ones = u32x4_t{IO::kOnes, IO::kOnes, IO::kOnes, IO::kOnes};
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (b < nblocks) {
          const u32x4_t ap = (BITS == 4 && !PERMUTED) ? a_perm_u4(av[b]) : av[b];
          if constexpr (ROWSUM) r = mfma16(av[b], ones, r, AT{});
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            uint32_t w0, w1;
            b_words(bv, t, b, w0, w1);
            d[t] = mfma16(ap, int_operand<FMT, AT>(w0, w1, vz), d[t], AT{});
          }
        }
      }
      if constexpr (GSM == GSM_CHANNEL) {
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = d[t];
        rsum = r;
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const IMeta m = make_imeta<FMT, AT>(mv[t][0]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = __builtin_fmaf(m.S, d[t][i], acc[t][i]);
            if constexpr (ROWSUM) v = __builtin_fmaf(-m.C, r[i], v);
            acc[t][i] = v;
          }
        }
      }
    } else {
      Meta mm[NT];
      if constexpr (GSM == GSM_CHANNEL) {
#pragma unroll
        for (int t = 0; t < NT; ++t) mm[t] = meta_ch[t];
      } else if constexpr (GSM == GSM_BIG) {
#pragma unroll
        for (int t = 0; t < NT; ++t) mm[t] = make_meta<FMT, AT>(mv[t][0]);
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (b < nblocks) {
          if constexpr (GSM == GSM_SMALL) {
#pragma unroll
            for (int t = 0; t < NT; ++t) mm[t] = make_meta<FMT, AT>(mv[t][b]);
          }
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            uint32_t w0, w1;
            b_words(bv, t, b, w0, w1);
            acc[t] = mfma16(av[b], dequant_operand<FMT, AT>(w0, w1, mm[t], vz), acc[t], AT{});
          }
        }
      }
    }
  };

  // Consume ring slot dc.  (ATX: piece (row r, k chunk c) of the step is MFMA block c/4,
  // lane (c%4)*16 + r; the row index is XOR-swizzled with c so that neither the 16 lanes
  // writing one row nor the 64 lanes reading one block collide on LDS banks.  A wave's own
  // LDS accesses complete in order, so the tile is rewritten each step without a barrier.)
  __shared__ u32x4_t lds_at[ATX ? WPB : 1][4 * 64];
  auto compute = [&](auto dc) __attribute__((always_inline)) {
    constexpr int d = decltype(dc)::value;
    if constexpr (ATX) {
      constexpr bool PERM = BITS == 4 && INT_B;
      const int c = lane & 15;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = 4 * b + (lane >> 4);
        lds_at[wave][(c >> 2) * 64 + (c & 3) * 16 + (r ^ c)] = PERM ? a_perm_u4(ra[d][b]) : ra[d][b];
      }
      u32x4_t av[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) av[b] = lds_at[wave][b * 64 + lg * 16 + (ln ^ (b * 4 + lg))];
      compute_regs(av, rb[d], rm[d], 4, std::integral_constant<bool, PERM>{});
    } else {
      compute_regs(ra[d], rb[d], rm[d], 4, std::false_type{});
    }
  };

  // ---- main loop ---------------------------------------------------------------------------
  // Step j lives in slot j % DEPTH; its weights are issued DEPTH-1 steps ahead, its
  // activations ALEAD steps ahead.  Each trip issues the activations before the weights so
  // that waiting for step j's activations never waits for a younger step's weights.
  // Prefetches past the last step are clamped to it (an L2 hit into a slot that is never
  // consumed); the last nsteps % DEPTH steps run after the loop.
  const int nsteps = max(s_end - s_begin, 0);
  if (nsteps > 0) {
    const int last = s_end - 1;
    static_for<ALEAD>([&](auto dc) { load_a(min(s_begin + (int)dc, last), dc); });
    static_for<DEPTH - 1>([&](auto dc) { load_b(min(s_begin + (int)dc, last), dc); });
    const int full_trips = nsteps / DEPTH;
    int s = s_begin;
    for (int i = 0; i < full_trips; ++i, s += DEPTH) {
      static_for<DEPTH>([&](auto dc) {
        constexpr int d = decltype(dc)::value;
        load_a(min(s + d + ALEAD, last), std::integral_constant<int, (d + ALEAD) % DEPTH>{});
        load_b(min(s + d + DEPTH - 1, last), std::integral_constant<int, (d + DEPTH - 1) % DEPTH>{});
        compute(dc);
      });
    }
    const int rem = nsteps - full_trips * DEPTH;
    static_for<DEPTH - 1>([&](auto dc) {
      constexpr int d = decltype(dc)::value;
      if (d < rem) {
        if constexpr (d >= ALEAD) load_a(s + d, dc);
        compute(dc);
      }
    });
  }

  // ---- K tail ------------------------------------------------------------------------------
  if (do_tail) {
    const int nblocks = k_tail / 32;
    const int kt0 = total_full * 128;
    u32x4_t av[4];
    u32x4_t bv[NT][NL];
    MetaRaw mv[NT][RAWB];
#pragma unroll
    for (int b = 0; b < 4; ++b)
      av[b] = b < nblocks ? *reinterpret_cast<const u32x4_t*>(a_row + kt0 + 32 * b)
                          : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t n = (int64_t)col_tile(t) * 16 + ln;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (b < nblocks) {
          const int64_t k = kt0 + 32 * b + 8 * lg;
          if constexpr (BITS == 4) {
            bv[t][0][b] = bbase[layout_word_index(4, p.K, p.N, n, k)];
          } else {
            bv[t][b >> 1][(b & 1) * 2] = bbase[layout_word_index(8, p.K, p.N, n, k)];
            bv[t][b >> 1][(b & 1) * 2 + 1] = bbase[layout_word_index(8, p.K, p.N, n, k + 4)];
          }
        }
      }
      if constexpr (GSM == GSM_BIG) {
        mv[t][0] = load_meta_raw<FMT, AT>(p, meta_base, kt0 >> p.group_shift, (int)n);
      } else if constexpr (GSM == GSM_SMALL) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          mv[t][b] = b < nblocks ? load_meta_raw<FMT, AT>(p, meta_base, (kt0 + 32 * b + 8 * lg) >> p.group_shift,
                                                         (int)n)
                                 : MetaRaw{0u, 0u};
      }
    }
    compute_regs(av, bv, mv, nblocks, std::false_type{});
  }

  // channelwise integer-operand path: apply the column scale / zero point once
  if constexpr (INT_B && GSM == GSM_CHANNEL) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const IMeta m = make_imeta<FMT, AT>(load_meta_raw<FMT, AT>(p, meta_base, 0, col_tile(t) * 16 + ln));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = m.S * acc[t][i];
        if constexpr (ROWSUM) v = __builtin_fmaf(-m.C, rsum[i], v);
        acc[t][i] = v;
      }
    }
  }

  // ---- KSPLIT: add the waves' partial sums --------------------------------------------------
  if constexpr (KSPLIT && WPB > 1) {
    __shared__ f32x4_t red[WPB - 1][NT][64];
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) red[wave - 1][t][lane] = acc[t];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < WPB - 1; ++w)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] += red[w][t][lane];
    }
    if constexpr (MOE) {
      __syncthreads();  // the next part reuses red
      if (wave > 0) continue;
    } else {
      if (wave > 0) return;
    }
  }

  // ---- epilogue ----------------------------------------------------------------------------
  // NVFP4: alpha scales the accumulator (global scale with the exponent-bias fold); a MoE
  // bias under router weights is scaled by the global scale as passed, unfolded, as the
  // reference's epilogue and bias init do (moe sm70_marlin_gemm.cuh:3490-3503,
  // sm70_marlin_bias.cu:56-58)
  float gscale = 1.0f;
  if constexpr (FMT == FMT_NVFP4) gscale = p.global_scale[expert];
  const float alpha = FMT == FMT_NVFP4 ? __builtin_ldexpf(gscale, p.alpha_exp) : 1.0f;
  const uint16_t* bias = reinterpret_cast<const uint16_t*>(p.bias);
  uint16_t* cout = reinterpret_cast<uint16_t*>(p.c);
  auto finish = [&](int row, int col, float v, float w) __attribute__((always_inline)) {
    float o = v * alpha;
    if (bias != nullptr) {
      float bv = raw16_to_float(load_u16<AT>(bias, (int64_t)expert * p.N + bias_storage_index(col)),
                                AT{});
      if constexpr (MOE) {
        if (p.mul_topk) bv *= gscale;
      }
      o += bv;
    }
    if constexpr (MOE) {
      if (p.mul_topk) o *= w;
    }
    cout[(int64_t)row * p.N + col] = to_raw16(o, AT{});
  };

  if constexpr (GATED) {
    // both factors of an output are in this lane: round each as stage 1 would store it,
    // then silu_and_mul's rounding (splits == 1)
    auto stage1_value = [&](int col, float v, float w) __attribute__((always_inline)) {
      float o = v * alpha;
      if (bias != nullptr) {
        float bv = raw16_to_float(load_u16<AT>(bias, (int64_t)expert * p.N + bias_storage_index(col)),
                                  AT{});
        if (p.mul_topk) bv *= gscale;
        o += bv;
      }
      if (p.mul_topk) o *= w;
      return (uint32_t)to_raw16(o, AT{});
    };
    const int half = p.N >> 1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int id = __shfl(row_id, lg * 4 + e);
      const float w = __shfl(route_w, part * 16 + lg * 4 + e);
      if (id >= 0) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = col_tile(t) * 16 + ln;
          const uint32_t g = stage1_value(col, acc[t][e], w);
          const uint32_t u = stage1_value(col_tile(t + 2) * 16 + ln, acc[t + 2][e], w);
          cout[(int64_t)id * half + col] = to_raw16(silu_mul1<AT>(g, u), AT{});
        }
      }
    }
    continue;
  }
  if constexpr (MOE) {
    // accumulator row lg*4+e belongs to the route held by lane lg*4+e (splits == 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int id = __shfl(row_id, lg * 4 + e);
      const float w = __shfl(route_w, part * 16 + lg * 4 + e);
      if (id >= 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) finish(id, col_tile(t) * 16 + ln, acc[t][e], w);
      }
    }
    continue;
  }

  if (nsplit == 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = lg * 4 + e;
        if (row < p.M) finish(row, col_tile(t) * 16 + ln, acc[t][e], 1.0f);
      }
    return;
  }

#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = lg * 4 + e;
      if (row < p.M)
        __hip_atomic_fetch_add(p.ws + (int64_t)row * p.N + col_tile(t) * 16 + ln, acc[t][e],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  // Same ordering argument as the tiled kernel: completed memory-side atomics, then the
  // arrival counter; the last arriver reads the sums back with atomic exchanges.
  wait_vm_all();
  int prev = 0;
  if (lane == 0)
    prev = __hip_atomic_fetch_add(p.counters + n_blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0);
  if (prev != nsplit - 1) return;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = lg * 4 + e;
      if (row < p.M) {
        const int col = col_tile(t) * 16 + ln;
        const float v = __hip_atomic_exchange(p.ws + (int64_t)row * p.N + col, 0.0f,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        finish(row, col, v, 1.0f);
      }
    }
  if (lane == 0)
    __hip_atomic_store(p.counters + n_blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }  // part loop
}

}  // namespace mmi
