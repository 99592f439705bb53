// stream_kernel.h -- multistage mixed-precision GEMM for 16..64-row blocks, gfx950.
//
// One workgroup = 4 wavefronts computes a BM x BN block (BN = 4 waves x NT n16 tiles); the
// waves share the BM activation rows and own disjoint columns.  Every operand of a K step
// (128 deep) is fetched three steps before it is multiplied, and nothing waits for more
// than the data it is about to use:
//   * weights (one dwordx4 of the chunk-major layout, device_common.h, per lane, tile and
//     1 KiB chunk), scale metadata and each wave's quarter of the activation tile are
//     loaded into a ring of three register sets;
//   * one step before use, each wave writes its quarter of the activation tile from the
//     ring into one of three LDS buffers (fragment-major with an XOR swizzle, so the staging
//     writes and every A-operand ds_read_b128 are conflict-free); one barrier per step
//     publishes it.  The quarter is loaded four whole rows per instruction.  (Activations
//     are not copied with global_load_lds_dwordx4: the compiler's wait-count insertion
//     cannot tell the buffers of such a ring apart and would wait for every pending load
//     before each LDS read.);
//   * slots and buffers are compile-time indices (static_for), the loop body is
//     branch-free, and prefetches past the last step are clamped to it, so the compiler's
//     vmcnt bookkeeping is exact on every trip; values that only a later step reads (fp4
//     scale bytes, 8-bit words before their lane swaps) are kept opaque until that step, so
//     the scheduler cannot pull their use up to the load;
//   * the 16x16 form issues the next step's loads a quarter per k32 block, between the
//     MFMAs; 256-column blocks also stage the following step's fragments a quarter at a
//     time, each right after the loads of the same quarter;
//   * split K (fp32 device-scope atomics) only up to 2^19 outputs (capi.hip);
//   * integer and fp8 weights with >= 128-deep groups (at most two m-tiles: the per-group
//     partial sums cost registers) or channelwise scales (any tile) use the integer-operand
//     path (device_common.h): codes feed the MFMA, the scale / zero point is applied to the
//     fp32 sums; the 4-bit activation permutation it needs is applied once, by the wave
//     that stages the fragment;
//   * the split-K protocol, the XCD-aware block order, the MoE row gather / scatter and the
//     epilogue are those of marlin_gemm_kernel (gemm_kernel.h).
#pragma once

#include "decode_kernel.h"

namespace mmi {

// GATED (MoE stage 1 with the SiLU-gated activation fused, splits == 1, 16x16 form): the
// workgroup's column block is 128 gate columns and the 128 matching up columns N/2 later;
// waves 0-1 stream the gate tiles and waves 2-3 the up tiles (4 KiB contiguous per step each,
// as in the plain kernel).  The up waves pass their finished, rounded outputs to the gate
// waves through LDS, which store silu(gate) * up into the [rows, N/2] output with the same
// rounding as the two-pass path (stage-1 output, then silu_and_mul).
template <int FMT, class AT, int BM, int NT, int GSM, bool MOE, bool GATED = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BM >= 128 ? 1 : 2, 8)))
void marlin_stream_kernel(const GemmParams p) {
  constexpr int MT = BM / 16;
  constexpr int BITS = fmt_bits(FMT);
  constexpr int BN = 4 * NT * 16;
  constexpr int NL = (BITS == 4) ? 1 : 2;  // 1 KiB chunk loads per tile per step
  constexpr int FRAGS = 4 * MT;             // A fragments per step (4 k32 blocks x MT)
  constexpr int FPW = MT;                   // A fragments staged by each wave
  constexpr int RAWB = (GSM == GSM_SMALL) ? 4 : 1;
  constexpr int D = 3;  // ring depth (register sets and LDS buffers)
  using IO = IntOperand<FMT, AT>;
  // 32x32x16 MFMAs (full rate on gfx950) for 128-row blocks and tile pairs; they also stage
  // the activations line by line (below).  Smaller blocks keep the 16x16x32 form and the
  // fragment-ordered loads, whose LDS addressing costs fewer registers at two waves per SIMD.
  constexpr bool M32 = BM >= 128 && NT % 2 == 0;
  constexpr int MT32 = M32 ? BM / 32 : 1;
  constexpr int NP = M32 ? NT / 2 : 1;
  // (the per-group scaling keeps a second set of MT x NT accumulators: at most two m-tiles;
  // the 32-row form has no room for row sums)
  constexpr bool INT_B = IO::kEnabled && GSM != GSM_SMALL && (MT <= 2 || GSM == GSM_CHANNEL) &&
                         !(M32 && IO::kNeedRowSum);
  constexpr bool ROWSUM = INT_B && IO::kNeedRowSum;

  __shared__ u32x4_t lds_a0[FRAGS * 64];
  __shared__ u32x4_t lds_a1[FRAGS * 64];
  __shared__ u32x4_t lds_a2[FRAGS * 64];
  __shared__ int lds_rows[BM];
  __shared__ float lds_w[BM];  // MoE: router weight of each block row (1 without mul_topk)
  __shared__ int lds_last;
  using Buf = u32x4_t[FRAGS * 64];
  auto buf = [&](auto dc) __attribute__((always_inline)) -> Buf& {
    constexpr int d = decltype(dc)::value;
    if constexpr (d == 0) return lds_a0;
    else if constexpr (d == 1) return lds_a1;
    else return lds_a2;
  };

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lg = lane >> 4;
  const int ln = lane & 15;
  const uint32_t vz = opaque_zero(p.zero);

  int split, n_blk, m_blk;
  decode_block(p, split, n_blk, m_blk);
  const int out_tile = m_blk * p.num_n_blocks + n_blk;

  int expert = 0;
  const uint16_t* a = reinterpret_cast<const uint16_t*>(p.a);
  if constexpr (MOE) {
    const int padded = p.num_post_pad[0];
    if (m_blk * p.moe_bs >= padded || m_blk >= p.expert_ids_numel) return;
    expert = p.expert_ids[m_blk];
    if (expert < 0) return;
    for (int r = tid; r < BM; r += 256) {
      int id = -1;
      const int si = m_blk * p.moe_bs + r;
      if (r < p.moe_bs && si < p.sorted_numel && si < padded) {
        id = p.sorted_ids[si];
        if (id < 0 || id >= p.valid_ids) id = -1;
      }
      lds_rows[r] = id;
      // (read once here, not once per output element in the epilogue)
      lds_w[r] = (p.mul_topk && id >= 0) ? p.topk_w[id] : 1.0f;
    }
    __syncthreads();
  }
  const int m0 = MOE ? 0 : m_blk * BM;

  // Activation staging: load i of this wave takes 16 bytes (8 k) at k offset 8*(lane%16) of
  // block row 4*(wave*FPW + i) + lane/16, so one load covers four whole 256-byte rows of the
  // step (8 full cache lines instead of 16 rows x 64 bytes).  Piece (row r, k chunk c) is
  // MFMA fragment (block c/4, m16 tile r/16), entry (c%4)*16 + r%16, the entry's low four
  // bits XOR-swizzled with c so that neither the 16 lanes writing one row nor the lanes
  // reading one fragment collide on LDS banks.
  auto a_unit = [&](int f, int g, int l16, int c) __attribute__((always_inline)) {
    return M32 ? f * 64 + g * 16 + (l16 ^ c) : f * 64 + g * 16 + l16;
  };
  const uint16_t* a_src[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    // (16x16 form: fragment f = wave + 4*i, k32 block f / MT, m16 tile f % MT, 16 rows x
    // 64 bytes per load)
    const int r = M32 ? (wave * FPW + i) * 4 + (lane >> 4) : ((wave + 4 * i) % MT) * 16 + ln;
    int64_t row;
    if constexpr (MOE) {
      const int id = lds_rows[r];
      row = id >= 0 ? id / p.top_k : 0;
    } else {
      row = min(m0 + r, p.M - 1);
    }
    a_src[i] = a + row * p.a_stride + (M32 ? 8 * (lane & 15) : 32 * ((wave + 4 * i) / MT) + 8 * lg);
  }
  auto stage_unit = [&](int i) __attribute__((always_inline)) {
    if constexpr (M32) {
      const int r = (wave * FPW + i) * 4 + (lane >> 4);
      const int c = lane & 15;
      return a_unit((c >> 2) * MT + (r >> 4), c & 3, r & 15, c);
    } else {
      return (wave + 4 * i) * 64 + lane;
    }
  };

  static_assert(!GATED || (MOE && !M32), "gated epilogue: MoE blocks, 16x16 form");
  const int tn0 = GATED ? (wave < 2 ? 0 : (p.N >> 5)) + n_blk * (BN / 32) + (wave & 1) * NT
                        : n_blk * (BN / 16) + wave * NT;
  const int64_t chunk_stride = (int64_t)(p.N >> 4) * 256;
  const uint32_t* bptr = p.b + (int64_t)expert * p.b_expert_stride + (int64_t)tn0 * 256 + lane * 4;
  const int64_t meta_base = (int64_t)expert * p.meta_expert_stride;

  const int total_full = p.K / 128;
  const int k_tail = p.K - total_full * 128;
  const int s_begin = split * p.steps_per_split;
  const int s_end = min(total_full, s_begin + p.steps_per_split);
  const bool do_tail = (k_tail != 0) && (split == p.splits - 1);

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f32x16_t acc32[MT32][NP];
#pragma unroll
  for (int i = 0; i < MT32; ++i)
#pragma unroll
    for (int t = 0; t < NP; ++t) acc32[i][t] = f32x16_t{};
  const int hi = (lane >> 4) & 1;  // M32: which tile of a pair holds this lane's column
  f32x4_t rsum[MT];  // channelwise integer-operand path: row sums over all of K
#pragma unroll
  for (int i = 0; i < MT; ++i) rsum[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  Meta meta_ch[NT];
  if constexpr (GSM == GSM_CHANNEL && !INT_B) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
      meta_ch[t] = make_meta<FMT, AT>(load_meta_raw<FMT, AT>(p, meta_base, 0, (tn0 + t) * 16 + ln));
  }

  u32x4_t ra[D][FPW];
  u32x4_t rb[D][NT][NL];
  MetaRaw rm[D][NT][RAWB];

  // Issue the loads of step s into ring slot dc: part q (0..3) takes the activation loads,
  // weight tiles and metadata whose index is q mod 4; part -1 takes all of them.
  auto load_part = [&](int s, auto dc, int q) __attribute__((always_inline)) {
    constexpr int d = decltype(dc)::value;
    const int k0 = s * 128;
#pragma unroll
    for (int i = 0; i < FPW; ++i)
      if (q < 0 || i % 4 == q) ra[d][i] = *reinterpret_cast<const u32x4_t*>(a_src[i] + k0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (q >= 0 && t % 4 != q) continue;
      const uint32_t* tp = bptr + t * 256 + (int64_t)s * NL * chunk_stride;
#pragma unroll
      for (int c = 0; c < NL; ++c)
        rb[d][t][c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(tp + c * chunk_stride));
      if constexpr (GSM == GSM_BIG) {
        rm[d][t][0] = load_meta_raw<FMT, AT>(p, meta_base, k0 >> p.group_shift, (tn0 + t) * 16 + ln);
      } else if constexpr (GSM == GSM_SMALL) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          rm[d][t][b] = load_meta_raw<FMT, AT>(p, meta_base, (k0 + 32 * b + 8 * lg) >> p.group_shift,
                                               (tn0 + t) * 16 + ln);
      }
    }
  };
  auto load = [&](int s, auto dc) __attribute__((always_inline)) { load_part(s, dc, -1); };

  // Write this wave's fragments of ring slot dc into LDS buffer dc.
  // (part q: the fragments whose index is q mod 4; part -1: all of them)
  auto stage_part = [&](auto dc, int q) __attribute__((always_inline)) {
    constexpr int d = decltype(dc)::value;
    Buf& lb = buf(dc);
#pragma unroll
    for (int i = 0; i < FPW; ++i)
      if (q < 0 || i % 4 == q) lb[stage_unit(i)] = (INT_B && BITS == 4) ? a_perm_u4(ra[d][i]) : ra[d][i];
  };
  auto stage = [&](auto dc) __attribute__((always_inline)) { stage_part(dc, -1); };

  auto b_words = [&](const u32x4_t (&bv)[NT][NL], int t, int b, uint32_t& w0, uint32_t& w1) __attribute__((always_inline)) {
    if constexpr (BITS == 4) {
      w0 = bv[t][0][b];
      w1 = 0;
    } else {
      w0 = bv[t][b >> 1][(b & 1) * 2];
      w1 = bv[t][b >> 1][(b & 1) * 2 + 1];
    }
  };

  // Multiply one step: activations from LDS buffer lb, weights / metadata from registers.
  // between(b) runs before k32 block b: the main loop issues a quarter of the next step's
  // loads there, so the memory pipeline takes them while the previous block's MFMAs run
  // (issued together right after the barrier, the four waves' loads queue for ~900 cycles)
  auto compute_core = [&](const Buf& lb, const u32x4_t (&bv)[NT][NL],
                          const MetaRaw (&mv)[NT][RAWB], int nblocks,
                          auto&& between) __attribute__((always_inline)) {
    if constexpr (M32) {
      // 32-row A operands straight from the 16x16 fragments (rows 32I + l%32, k-slice
      // 2h + l/32 of block b); B operands re-dealt from tile pairs with deal32().
      Meta mm[NP];
      if constexpr (!INT_B) {
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          if constexpr (GSM == GSM_CHANNEL) mm[q] = hi ? meta_ch[2 * q + 1] : meta_ch[2 * q];
          else mm[q] = make_meta<FMT, AT>(hi ? mv[2 * q + 1][0] : mv[2 * q][0]);
        }
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        between(b);
        if (b < nblocks) {
          u32x4_t a32[MT32][2];
#pragma unroll
          for (int i = 0; i < MT32; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              a32[i][h] = lb[a_unit(b * MT + 2 * i + hi, 2 * h + (lane >> 5), lane & 15,
                                    4 * b + 2 * h + (lane >> 5))];
#pragma unroll
          for (int q = 0; q < NP; ++q) {
            uint32_t x0, x1, y0, y1;
            b_words(bv, 2 * q, b, x0, x1);
            b_words(bv, 2 * q + 1, b, y0, y1);
            // 8-bit words opaque here: left visible, the scheduler moves the lane swaps of a
            // ring slot up to its loads, a trip early, and the wave waits for loads it has
            // just issued (cfg3 shape: 592 -> 552 us; 4-bit words: 422 -> 436 us at cfg2
            // M = 1024, so they stay visible)
            if constexpr (BITS == 8) asm volatile("" : "+v"(x0), "+v"(y0), "+v"(x1), "+v"(y1));
            uint32_t w0[2], w1[2] = {0u, 0u};
            deal32(x0, y0, w0[0], w0[1]);
            if constexpr (BITS == 8) deal32(x1, y1, w1[0], w1[1]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              u32x4_t bop;
              if constexpr (INT_B) bop = int_operand<FMT, AT>(w0[h], w1[h], vz);
              else bop = dequant_operand<FMT, AT>(w0[h], w1[h], mm[q], vz);
#pragma unroll
              for (int i = 0; i < MT32; ++i) acc32[i][q] = mfma32(a32[i][h], bop, acc32[i][q], AT{});
            }
          }
        }
      }
    } else if constexpr (INT_B) {
      f32x4_t d[MT][NT];
      f32x4_t r[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        r[i] = GSM == GSM_CHANNEL ? rsum[i] : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NT; ++t)
          d[i][t] = GSM == GSM_CHANNEL ? acc[i][t] : f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      const u32x4_t ones = u32x4_t{IO::kOnes, IO::kOnes, IO::kOnes, IO::kOnes};
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        between(b);
        if (b < nblocks) {
          u32x4_t af[MT];
#pragma unroll
          for (int i = 0; i < MT; ++i) af[i] = lb[a_unit(b * MT + i, lg, ln, 4 * b + lg)];
          if constexpr (ROWSUM) {
#pragma unroll
            for (int i = 0; i < MT; ++i) r[i] = mfma16(af[i], ones, r[i], AT{});
          }
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            uint32_t w0, w1;
            b_words(bv, t, b, w0, w1);
            const u32x4_t bop = int_operand<FMT, AT>(w0, w1, vz);
#pragma unroll
            for (int i = 0; i < MT; ++i) d[i][t] = mfma16(af[i], bop, d[i][t], AT{});
          }
        }
      }
      if constexpr (GSM == GSM_CHANNEL) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          rsum[i] = r[i];
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[i][t] = d[i][t];
        }
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const IMeta m = make_imeta<FMT, AT>(mv[t][0]);
#pragma unroll
          for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float v = __builtin_fmaf(m.S, d[i][t][e], acc[i][t][e]);
              if constexpr (ROWSUM) v = __builtin_fmaf(-m.C, r[i][e], v);
              acc[i][t][e] = v;
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
        between(b);
        if (b < nblocks) {
          if constexpr (GSM == GSM_SMALL) {
#pragma unroll
            for (int t = 0; t < NT; ++t) mm[t] = make_meta<FMT, AT>(mv[t][b]);
          }
          u32x4_t af[MT];
#pragma unroll
          for (int i = 0; i < MT; ++i) af[i] = lb[a_unit(b * MT + i, lg, ln, 4 * b + lg)];
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            uint32_t w0, w1;
            b_words(bv, t, b, w0, w1);
            const u32x4_t bop = dequant_operand<FMT, AT>(w0, w1, mm[t], vz);
#pragma unroll
            for (int i = 0; i < MT; ++i) acc[i][t] = mfma16(af[i], bop, acc[i][t], AT{});
          }
        }
      }
    }
  };

  // ---- main loop ---------------------------------------------------------------------------
  // Step j: registers in slot j % 3, activations in LDS buffer j % 3.  Trip j issues the
  // loads of step j+2, stages the activations of step j+1, multiplies step j, then one
  // barrier: buffer (j+1) % 3 is published and nobody still reads the buffer the next trip
  // overwrites.
  const int nsteps = max(s_end - s_begin, 0);
  if (nsteps > 0) {
    const int last = s_end - 1;
    load(s_begin, std::integral_constant<int, 0>{});
    load(min(s_begin + 1, last), std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 0>{});
    __syncthreads();
    const int full_trips = nsteps / D;
    int s = s_begin;
    auto trip = [&](auto dc) __attribute__((always_inline)) {
      constexpr int d = decltype(dc)::value;
      // 16x16 form: the next step's loads go out a quarter per k32 block, between the
      // blocks' MFMAs (cfg2 M=128: 101 -> 94 us; MoE stage 1 at T=2048: 706 -> 667 us).  The
      // 128-row 32x32 form issues them up front (spread: 418 -> 436 us at M=1024).
      constexpr bool kSpread = !M32;
      // 256-column blocks also stage the next step's fragments a quarter per k32 block, each
      // right after the matching quarter of loads, so that fragment i waits for a load
      // issued a whole trip before instead of the last quarter's (MoE stage 1 + 2 at
      // T = 2048: 1080 -> 1051 us; 128-column blocks measured no better)
      constexpr bool kSpreadStage = kSpread && NT >= 4;
      if constexpr (!kSpread) load(min(s + d + 2, last), std::integral_constant<int, (d + 2) % D>{});
      if constexpr (!kSpreadStage) stage(std::integral_constant<int, (d + 1) % D>{});
      compute_core(buf(dc), rb[d], rm[d], 4, [&](int q) __attribute__((always_inline)) {
        if constexpr (kSpread) {
          __builtin_amdgcn_sched_barrier(0);
          load_part(min(s + d + 2, last), std::integral_constant<int, (d + 2) % D>{}, q);
          if constexpr (kSpreadStage) stage_part(std::integral_constant<int, (d + 1) % D>{}, q);
          __builtin_amdgcn_sched_barrier(0);
        }
      });
      __syncthreads();
    };
    for (int i = 0; i < full_trips; ++i, s += D) static_for<D>(trip);
    const int rem = nsteps - full_trips * D;
    // remaining steps: s, s+1 (slots 0, 1); their loads and staging were issued above
    if (rem > 0) {
      stage(std::integral_constant<int, 1>{});
      compute_core(lds_a0, rb[0], rm[0], 4, [](int) {});
      __syncthreads();
      if (rem > 1) compute_core(lds_a1, rb[1], rm[1], 4, [](int) {});
    }
  }

  // ---- K tail: (K % 128) / 32 blocks, read word by word through the layout map -----------
  if (do_tail) {
    const int nblocks = k_tail / 32;
    const int kt0 = total_full * 128;
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      const int b = M32 ? (lane & 15) >> 2 : (wave + 4 * i) / MT;
      u32x4_t v = b < nblocks ? *reinterpret_cast<const u32x4_t*>(a_src[i] + kt0)
                              : u32x4_t{0u, 0u, 0u, 0u};
      lds_a2[stage_unit(i)] = (INT_B && BITS == 4) ? a_perm_u4(v) : v;
    }
    u32x4_t bw[NT][NL];
    MetaRaw raw[NT][RAWB];
    const uint32_t* base = p.b + (int64_t)expert * p.b_expert_stride;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t n = (int64_t)(tn0 + t) * 16 + ln;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (b < nblocks) {
          const int64_t k = kt0 + 32 * b + 8 * lg;
          if constexpr (BITS == 4) {
            bw[t][0][b] = base[layout_word_index(4, p.K, p.N, n, k)];
          } else {
            bw[t][b >> 1][(b & 1) * 2] = base[layout_word_index(8, p.K, p.N, n, k)];
            bw[t][b >> 1][(b & 1) * 2 + 1] = base[layout_word_index(8, p.K, p.N, n, k + 4)];
          }
        }
      }
      if constexpr (GSM == GSM_BIG) {
        raw[t][0] = load_meta_raw<FMT, AT>(p, meta_base, kt0 >> p.group_shift, (int)n);
      } else if constexpr (GSM == GSM_SMALL) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          raw[t][b] = b < nblocks ? load_meta_raw<FMT, AT>(p, meta_base,
                                                          (kt0 + 32 * b + 8 * lg) >> p.group_shift,
                                                          (int)n)
                                  : MetaRaw{0u, 0u};
      }
    }
    __syncthreads();
    compute_core(lds_a2, bw, raw, nblocks, [](int) {});
  }

  if constexpr (INT_B && GSM == GSM_CHANNEL && M32) {
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const IMeta m = make_imeta<FMT, AT>(load_meta_raw<FMT, AT>(p, meta_base, 0, (tn0 + 2 * q + hi) * 16 + ln));
#pragma unroll
      for (int i = 0; i < MT32; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc32[i][q][v] *= m.S;
    }
  } else if constexpr (INT_B && GSM == GSM_CHANNEL) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const IMeta m = make_imeta<FMT, AT>(load_meta_raw<FMT, AT>(p, meta_base, 0, (tn0 + t) * 16 + ln));
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = m.S * acc[i][t][e];
          if constexpr (ROWSUM) v = __builtin_fmaf(-m.C, rsum[i][e], v);
          acc[i][t][e] = v;
        }
    }
  }

  // ---- epilogue --------------------------------------------------------------------------
  // NVFP4: alpha scales the accumulator (global scale with the exponent-bias fold); a MoE
  // bias under router weights is scaled by the global scale as passed, unfolded, as the
  // reference's epilogue and bias init do (moe sm70_marlin_gemm.cuh:3490-3503,
  // sm70_marlin_bias.cu:56-58)
  float gscale = 1.0f;
  if constexpr (FMT == FMT_NVFP4) gscale = p.global_scale[expert];
  const float alpha = FMT == FMT_NVFP4 ? __builtin_ldexpf(gscale, p.alpha_exp) : 1.0f;
  const uint16_t* bias = reinterpret_cast<const uint16_t*>(p.bias);
  uint16_t* cout = reinterpret_cast<uint16_t*>(p.c);

  auto out_row = [&](int r) __attribute__((always_inline)) -> int64_t {  // -1: not stored
    if constexpr (MOE) {
      return lds_rows[r];
    } else {
      return (m0 + r < p.M) ? (int64_t)(m0 + r) : -1;
    }
  };

  auto finish = [&](int r, int col, float v) __attribute__((always_inline)) {
    const int64_t orow = out_row(r);
    if (orow < 0) return;
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
      if (p.mul_topk) o *= lds_w[r];
    }
    cout[orow * p.N + col] = to_raw16(o, AT{});
  };

  // every output this lane holds: (block row, column, value)
  auto for_out = [&](auto&& f) __attribute__((always_inline)) {
    if constexpr (M32) {
#pragma unroll
      for (int i = 0; i < MT32; ++i)
#pragma unroll
        for (int q = 0; q < NP; ++q)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            f(32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3), (tn0 + 2 * q) * 16 + (lane & 31),
              acc32[i][q][v]);
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) f(i * 16 + lg * 4 + e, (tn0 + t) * 16 + ln, acc[i][t][e]);
    }
  };

  if constexpr (GATED) {
    // value of one output as the two-pass path stores it (finish() without the store)
    auto stage1_value = [&](int r, int col, float v) __attribute__((always_inline)) {
      float o = v * alpha;
      if (bias != nullptr) {
        float bv = raw16_to_float(load_u16<AT>(bias, (int64_t)expert * p.N + bias_storage_index(col)),
                                  AT{});
        if (p.mul_topk) bv *= gscale;
        o += bv;
      }
      if (p.mul_topk) o *= lds_w[r];
      return (uint32_t)to_raw16(o, AT{});
    };
    // Gate wave w and up wave w + 2 hold the two factors of the same outputs.  Each finishes
    // half of them: the gate wave the first half (it receives those up values), the up wave
    // the second half (it receives those gate values), so the SiLU work is spread over all
    // four waves.
    constexpr int PER = MT * NT * 4;  // outputs per lane
    constexpr int HALF = PER / 2;
    uint16_t* xch = reinterpret_cast<uint16_t*>(lds_a0);  // [2 pairs][PER][64]
    static_assert(2 * PER * 64 * 2 <= (int)sizeof(lds_a0), "exchange fits the staging buffer");
    const bool up = wave >= 2;
    uint16_t* mine = xch + (wave & 1) * PER * 64;  // this pair's exchange area
    __syncthreads();  // every wave is done reading the staging buffers
    {
      int j = 0;
      for_out([&](int r, int col, float v) __attribute__((always_inline)) {
        // the gate wave hands over its second half, the up wave its first half
        if (up ? j < HALF : j >= HALF) {
          const int64_t orow = out_row(r);
          mine[j * 64 + lane] = orow >= 0 ? (uint16_t)stage1_value(r, col, v) : 0;
        }
        ++j;
      });
    }
    __syncthreads();
    {
      const int half = p.N >> 1;
      int j = 0;
      for_out([&](int r, int col, float v) __attribute__((always_inline)) {
        const bool own = up ? j >= HALF : j < HALF;
        const int jj = j++;
        if (!own) return;
        const int64_t orow = out_row(r);
        if (orow < 0) return;
        const uint32_t other = mine[jj * 64 + lane];
        const uint32_t self = stage1_value(r, col, v);
        const uint32_t g = up ? other : self;
        const uint32_t u = up ? self : other;
        cout[orow * half + (up ? col - half : col)] = to_raw16(silu_mul1<AT>(g, u), AT{});
      });
    }
    return;
  }

  if (p.splits == 1) {
    for_out([&](int r, int col, float v) __attribute__((always_inline)) { finish(r, col, v); });
    return;
  }

  // split-K (same protocol as marlin_gemm_kernel)
  for_out([&](int r, int col, float v) __attribute__((always_inline)) {
    const int64_t orow = out_row(r);
    if (orow >= 0)
      __hip_atomic_fetch_add(p.ws + orow * p.N + col, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  });
  wait_vm_all();
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(p.counters + out_tile, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    lds_last = (prev == p.splits - 1);
  }
  __syncthreads();
  if (!lds_last) return;
  for_out([&](int r, int col, float) __attribute__((always_inline)) {
    const int64_t orow = out_row(r);
    if (orow >= 0) {
      const float v = __hip_atomic_exchange(p.ws + orow * p.N + col, 0.0f, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
      finish(r, col, v);
    }
  });
  if (tid == 0)
    __hip_atomic_store(p.counters + out_tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mmi
