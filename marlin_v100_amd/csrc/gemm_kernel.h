// gemm_kernel.h -- gfx950 mixed-precision GEMM mainloop shared by the dense and MoE ops.
//
// Work decomposition (one workgroup = 4 wavefronts = 256 threads):
//   * a workgroup owns a BM x BN output block, BN = 4 waves x NT n16-tiles x 16 columns;
//     all four waves share the BM activation rows and own disjoint columns, so no weight
//     is dequantized twice;
//   * K advances in steps of CH chunks (128*CH deep).  Activation rows for the step are
//     copied straight into LDS with global_load_lds_dwordx4 (no VGPR staging), laid out
//     fragment-major so every ds_read_b128 of an MFMA A operand is conflict-free;
//   * weights never touch LDS: each lane loads its dwordx4s of the chunk-major layout
//     (device_common.h), dequantizes in registers and feeds v_mfma_f32_16x16x32;
//   * the next step's activations, weights and scale metadata are in flight while the
//     current step computes (two LDS arrays / register sets, loop unrolled by two);
//   * split-K partitions the K steps; partial sums go to an fp32 workspace with device-scope
//     atomics, the last workgroup to finish an output block (per-block arrival counter)
//     applies the epilogue and resets its workspace slice and counter to zero, so the
//     workspace needs no clearing between calls;
//   * dense tiles are visited in an XCD-aware grouped order: consecutive workgroup ids go
//     to different XCDs, so ids are remapped such that each XCD works on a compact group
//     of output tiles and reuses the activation and weight slabs from its own L2.
// MoE (reference sm70_marlin_gemm.cuh:3591-3686): a workgroup's rows are one moe block of
// expert-sorted route ids; A rows are gathered as id / top_k, C rows scattered to id.
#pragma once

#include "device_common.h"

namespace mmi {

struct GemmParams {
  const void* a;
  int64_t a_stride;  // elements between rows of A
  void* c;           // output rows of N elements
  const uint32_t* b;
  int64_t b_expert_stride;  // words per expert (MoE)
  const void* scales;       // [E][G][N]
  const void* zeros;        // [E][G][N] float zero points (same dtype as A) or null
  int64_t meta_expert_stride;  // G*N
  const void* bias;            // [E][N] permuted, or null
  const float* global_scale;   // NVFP4: [E]
  int alpha_exp;               // alpha = ldexp(global_scale[e], alpha_exp)
  int M, N, K;
  int group_shift;  // log2(group size) for grouped modes
  int splits;
  int steps_per_split;
  int main_blocks;  // decode kernel: the last main_blocks blocks take all of K unsplit; the
                    // blocks before them split K `splits` ways (0: every block splits)
  int num_n_blocks;
  int num_m_blocks;
  int xcd_group_m;  // m-blocks per group in the XCD-aware order (0: plain order)
  int xcd_interleave;  // MoE: deal whole groups to the XCDs in turn (needs splits == 1)
  float* ws;
  int* counters;
  // MoE
  const int* sorted_ids;
  int sorted_numel;
  const int* expert_ids;
  int expert_ids_numel;
  const int* num_post_pad;
  const float* topk_w;
  int top_k;
  int moe_bs;
  int mul_topk;
  int valid_ids;  // size_m * top_k
  int zero;       // always 0: source of an opaque VGPR zero (opaque_zero())
};

// Group-size modes.
enum { GSM_CHANNEL = 0, GSM_BIG = 1, GSM_SMALL = 2 };

constexpr int kNumXcd = 8;

template <class AT>
__device__ __forceinline__ uint32_t load_u16(const void* p, int64_t idx) {
  return (uint32_t)(reinterpret_cast<const uint16_t*>(p)[idx]);
}

template <int FMT, class AT>
__device__ __forceinline__ MetaRaw load_meta_raw(const GemmParams& p, int64_t base, int group,
                                                 int col) {
  const int64_t idx = base + (int64_t)group * p.N;
  if constexpr (FMT == FMT_NVFP4) {
    // NVFP4 scales are stored with a [0,2,1,3] shuffle per 4 columns
    // (marlin_utils_fp4.py:83-86); the shuffle is its own inverse.
    const int sc = (col & ~3) | ((col & 1) << 1) | ((col & 2) >> 1);
    return MetaRaw{reinterpret_cast<const uint8_t*>(p.scales)[idx + sc], 0u};
  } else if constexpr (FMT == FMT_MXFP4) {
    return MetaRaw{reinterpret_cast<const uint8_t*>(p.scales)[idx + col], 0u};
  } else if constexpr (fmt_has_zp(FMT)) {
    // a float zero point, or (integer-zero formats) the 16-bit code the launcher expanded
    // from the caller's packed int32 words into the same [G, N] layout
    const int64_t e = idx + col;
    const uint32_t z = load_u16<AT>(p.zeros, e);
    return MetaRaw{load_u16<AT>(p.scales, e), z};
  } else {
    return MetaRaw{load_u16<AT>(p.scales, idx + col), 0u};
  }
}

__device__ __forceinline__ void lds_dma16(const void* gptr, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)lds_wave_base,
                                   16, 0, 0);
}

__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Keeps the compiler from reordering memory instructions across this point (emits nothing).
// The vmcnt a consumer waits for is counted from the issue order of the loads, so a ring of
// loads only keeps its depth if every path into the loop issues them in the same order.
__device__ __forceinline__ void issue_order() { asm volatile("" ::: "memory"); }

// Workgroup id -> (split, n block, m block).  Dense launches use the XCD-aware grouped
// order when p.xcd_group_m > 0: each XCD takes a contiguous range of the grouped order.
// MoE launches with p.xcd_interleave set (splits == 1) deal whole groups (xcd_group_m moe
// blocks x all n blocks) to the XCDs in turn: the moe blocks of one expert then share the
// expert's weight slab, and the group's activation rows, in one L2, and the groups of dead
// moe blocks at the end of the padded grid spread over all XCDs.
__device__ __forceinline__ void decode_block(const GemmParams& p, int& split, int& n_blk,
                                             int& m_blk) {
  int id = blockIdx.x;
  const int total = gridDim.x;
  if (p.xcd_interleave > 0) {
    const int gm_full = p.xcd_group_m;
    const int per_group = gm_full * p.num_n_blocks;
    const int full = total - total % (kNumXcd * per_group);
    if (id < full) {
      const int j = id / kNumXcd;
      id = ((j / per_group) * kNumXcd + id % kNumXcd) * per_group + j % per_group;
    }
    const int g = id / per_group;
    const int first_m = g * gm_full;
    const int gm = min(p.num_m_blocks - first_m, gm_full);
    const int in = id - g * per_group;
    split = 0;
    m_blk = first_m + in % gm;
    n_blk = in / gm;
    return;
  }
  if (p.xcd_group_m > 0) {
    const int full = total - total % kNumXcd;
    if (id < full) {
      const int per = full / kNumXcd;
      id = (id % kNumXcd) * per + id / kNumXcd;
    }
  }
  split = id % p.splits;
  const int tile = id / p.splits;
  if (p.xcd_group_m > 0) {
    const int gm_full = p.xcd_group_m;
    const int per_group = gm_full * p.num_n_blocks;
    const int g = tile / per_group;
    const int first_m = g * gm_full;
    const int gm = min(p.num_m_blocks - first_m, gm_full);
    const int in = tile - g * per_group;
    m_blk = first_m + in % gm;
    n_blk = in / gm;
  } else {
    n_blk = tile % p.num_n_blocks;
    m_blk = tile / p.num_n_blocks;
  }
}

// Waves per SIMD the register allocation must leave room for: the small-M (weight
// streaming) tiles need many waves in flight, the 128-row tiles trade occupancy for
// accumulators.
template <int BM>
constexpr int waves_per_eu() {
  return BM <= 32 ? 4 : (BM <= 64 ? 2 : 1);
}

template <int FMT, class AT, int BM, int NT, int CH, int GSM, bool MOE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(waves_per_eu<BM>(), 8)))
void marlin_gemm_kernel(const GemmParams p) {
  constexpr int MT = BM / 16;
  constexpr int BITS = fmt_bits(FMT);
  constexpr int BN = 4 * NT * 16;
  constexpr int NB = 4 * CH;                      // k32 blocks per step
  constexpr int KS = 128 * CH;                    // k per step
  constexpr int NL = (BITS == 4) ? CH : 2 * CH;   // 1 KiB chunk loads per tile per step
  constexpr int FRAGS = NB * MT;                  // A fragments per step
  constexpr int FPW = FRAGS / 4;                  // A fragments copied by each wave
  static_assert(FRAGS % 4 == 0, "fragments split evenly over 4 waves");
  constexpr int RAWB = (GSM == GSM_SMALL) ? NB : (GSM == GSM_BIG ? CH : 1);

  // Two distinct LDS arrays (not one [2][...] array): the next step's global->LDS copies
  // target the other array, and the compiler can only prove they do not alias the current
  // step's ds_reads -- and so keep them in flight -- when the objects are distinct.
  __shared__ u32x4_t lds_a0[FRAGS * 64];
  __shared__ u32x4_t lds_a1[FRAGS * 64];
  __shared__ int lds_rows[BM];
  __shared__ float lds_w[BM];  // MoE: router weight of each block row (1 without mul_topk)
  __shared__ int lds_last;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lg = lane >> 4;  // lane group: k-slice 8*lg inside a 32-deep block
  const int ln = lane & 15;  // column (B) / row (A) inside a 16-wide fragment
  const uint32_t vz = opaque_zero(p.zero);

  int split, n_blk, m_blk;
  decode_block(p, split, n_blk, m_blk);
  const int out_tile = m_blk * p.num_n_blocks + n_blk;

  int expert = 0;
  // activations as raw 16-bit words (AT is a tag type, not the element type)
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

  // ---- activation rows this wave copies into LDS: fragments f = wave + 4*i --------------
  // fragment f covers k32 block f / MT and m16 tile f % MT of the step
  const uint16_t* a_src[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = wave + 4 * i;
    const int b = f / MT;
    const int mt = f % MT;
    const int r = mt * 16 + ln;
    int64_t row;
    if constexpr (MOE) {
      const int id = lds_rows[r];
      row = id >= 0 ? id / p.top_k : 0;
    } else {
      row = min(m0 + r, p.M - 1);
    }
    a_src[i] = a + row * p.a_stride + 32 * b + 8 * lg;
  }

  // ---- weight / metadata addressing ------------------------------------------------------
  const int tn0 = n_blk * (BN / 16) + wave * NT;  // first n16 tile of this wave
  // chunk c of tile t is at word (c * tiles + t) * 256 (chunk-major layout)
  const int64_t chunk_stride = (int64_t)(p.N >> 4) * 256;
  const uint32_t* bptr = p.b + (int64_t)expert * p.b_expert_stride + (int64_t)tn0 * 256 + lane * 4;
  const int64_t meta_base = (int64_t)expert * p.meta_expert_stride;

  const int total_full = p.K / KS;
  const int k_tail = p.K - total_full * KS;
  const int s_begin = split * p.steps_per_split;
  const int s_end = min(total_full, s_begin + p.steps_per_split);
  const bool do_tail = (k_tail != 0) && (split == p.splits - 1);

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Channelwise metadata is loop invariant.
  Meta meta_ch[NT];
  if constexpr (GSM == GSM_CHANNEL) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
      meta_ch[t] = make_meta<FMT, AT>(load_meta_raw<FMT, AT>(p, meta_base, 0, (tn0 + t) * 16 + ln));
  }

  auto load_step = [&](int s, u32x4_t (&lds)[FRAGS * 64], u32x4_t (&bw)[NT][NL],
                       MetaRaw (&raw)[NT][RAWB]) {
    const int k0 = s * KS;
    // activations -> LDS
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      const int f = wave + 4 * i;
      lds_dma16(a_src[i] + k0, &lds[f * 64]);
    }
    // weights: NL consecutive 1 KiB chunks of each tile
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t* tp = bptr + t * 256 + (int64_t)s * NL * chunk_stride;
#pragma unroll
      for (int c = 0; c < NL; ++c)
        bw[t][c] = *reinterpret_cast<const u32x4_t*>(tp + c * chunk_stride);
    }
    // metadata
    if constexpr (GSM == GSM_BIG) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int c = 0; c < CH; ++c)
          raw[t][c] = load_meta_raw<FMT, AT>(p, meta_base, (k0 + 128 * c) >> p.group_shift,
                                             (tn0 + t) * 16 + ln);
    } else if constexpr (GSM == GSM_SMALL) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int b = 0; b < NB; ++b)
          raw[t][b] = load_meta_raw<FMT, AT>(p, meta_base, (k0 + 32 * b + 8 * lg) >> p.group_shift,
                                             (tn0 + t) * 16 + ln);
    }
  };

  auto compute_step = [&](const u32x4_t (&lds)[FRAGS * 64], const u32x4_t (&bw)[NT][NL],
                          const MetaRaw (&raw)[NT][RAWB], int nblocks) {
    Meta mm[NT];
    if constexpr (GSM == GSM_CHANNEL) {
#pragma unroll
      for (int t = 0; t < NT; ++t) mm[t] = meta_ch[t];
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b < nblocks) {
        if constexpr (GSM == GSM_SMALL) {
#pragma unroll
          for (int t = 0; t < NT; ++t) mm[t] = make_meta<FMT, AT>(raw[t][b]);
        } else if constexpr (GSM == GSM_BIG) {
          if ((b & 3) == 0) {
#pragma unroll
            for (int t = 0; t < NT; ++t) mm[t] = make_meta<FMT, AT>(raw[t][b >> 2]);
          }
        }
        u32x4_t af[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) af[i] = lds[(b * MT + i) * 64 + lane];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          uint32_t w0, w1;
          if constexpr (BITS == 4) {
            w0 = bw[t][b >> 2][b & 3];
            w1 = 0;
          } else {
            w0 = bw[t][b >> 1][(b & 1) * 2];
            w1 = bw[t][b >> 1][(b & 1) * 2 + 1];
          }
          const u32x4_t bop = dequant_operand<FMT, AT>(w0, w1, mm[t], vz);
#pragma unroll
          for (int i = 0; i < MT; ++i) acc[i][t] = mfma16(af[i], bop, acc[i][t], AT{});
        }
      }
    }
  };

  // ---- main loop over full steps, ping-pong between two register / LDS sets ---------------
  if (s_begin < s_end) {
    u32x4_t b0[NT][NL], b1[NT][NL];
    MetaRaw r0[NT][RAWB], r1[NT][RAWB];
    load_step(s_begin, lds_a0, b0, r0);
    wait_vm_all();
    __syncthreads();
    int s = s_begin;
    while (true) {
      bool more = s + 1 < s_end;
      if (more) load_step(s + 1, lds_a1, b1, r1);
      compute_step(lds_a0, b0, r0, NB);
      wait_vm_all();
      __syncthreads();
      if (!more) break;
      ++s;
      more = s + 1 < s_end;
      if (more) load_step(s + 1, lds_a0, b0, r0);
      compute_step(lds_a1, b1, r1, NB);
      wait_vm_all();
      __syncthreads();
      if (!more) break;
      ++s;
    }
  }

  // ---- K tail: (K % KS) / 32 blocks, read word by word through the layout map ------------
  if (do_tail) {
    const int nblocks = k_tail / 32;
    const int kt0 = total_full * KS;
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      const int f = wave + 4 * i;
      const int b = f / MT;
      if (b < nblocks) lds_dma16(a_src[i] + kt0, &lds_a0[f * 64]);
    }
    u32x4_t bw[NT][NL];
    MetaRaw raw[NT][RAWB];
    const uint32_t* base = p.b + (int64_t)expert * p.b_expert_stride;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t n = (int64_t)(tn0 + t) * 16 + ln;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b < nblocks) {
          const int64_t k = kt0 + 32 * b + 8 * lg;
          if constexpr (BITS == 4) {
            bw[t][b >> 2][b & 3] = base[layout_word_index(4, p.K, p.N, n, k)];
          } else {
            bw[t][b >> 1][(b & 1) * 2] = base[layout_word_index(8, p.K, p.N, n, k)];
            bw[t][b >> 1][(b & 1) * 2 + 1] = base[layout_word_index(8, p.K, p.N, n, k + 4)];
          }
        }
      }
      if constexpr (GSM == GSM_BIG) {
#pragma unroll
        for (int c = 0; c < CH; ++c)
          raw[t][c] = 4 * c < nblocks ? load_meta_raw<FMT, AT>(p, meta_base,
                                                              (kt0 + 128 * c) >> p.group_shift,
                                                              (int)n)
                                      : MetaRaw{0u, 0u};
      } else if constexpr (GSM == GSM_SMALL) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
          raw[t][b] = b < nblocks ? load_meta_raw<FMT, AT>(p, meta_base,
                                                          (kt0 + 32 * b + 8 * lg) >> p.group_shift,
                                                          (int)n)
                                  : MetaRaw{0u, 0u};
      }
    }
    wait_vm_all();
    __syncthreads();
    compute_step(lds_a0, bw, raw, nblocks);
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

  auto out_row = [&](int r) -> int64_t {  // -1 when the row is not stored
    if constexpr (MOE) {
      return lds_rows[r];
    } else {
      return (m0 + r < p.M) ? (int64_t)(m0 + r) : -1;
    }
  };

  auto finish = [&](int r, int col, float v) {
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

  if (p.splits == 1) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          finish(i * 16 + lg * 4 + e, (tn0 + t) * 16 + ln, acc[i][t][e]);
    return;
  }

  // split-K: accumulate into the fp32 workspace, last arriver finishes the block.
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t orow = out_row(i * 16 + lg * 4 + e);
        if (orow >= 0)
          __hip_atomic_fetch_add(p.ws + orow * p.N + (tn0 + t) * 16 + ln, acc[i][t][e],
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
  // Ordering without an agent-scope fence (which on gfx950 writes back and invalidates the
  // whole L2): the partial sums are device-scope atomics performed at the memory side, so
  // once they have completed (vmcnt drained) every later atomic on any XCD observes them.
  // The arrival counter is bumped only after that, and the last arriver reads the sums with
  // atomic exchanges, which cannot be served from a stale cache line.
  wait_vm_all();
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(p.counters + out_tile, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    lds_last = (prev == p.splits - 1);
  }
  __syncthreads();
  if (!lds_last) return;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = i * 16 + lg * 4 + e;
        const int64_t orow = out_row(r);
        if (orow >= 0) {
          const int col = (tn0 + t) * 16 + ln;
          const float v = __hip_atomic_exchange(p.ws + orow * p.N + col, 0.0f, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
          finish(r, col, v);
        }
      }
  if (tid == 0)
    __hip_atomic_store(p.counters + out_tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mmi
