// aux_kernels.hip -- dequantize (inspection op), moe_align_block_size, moe_sum and the MoE
// SiLU-and-multiply activation.
#include <algorithm>

#include "gemm_kernel.h"
#include "host_common.h"

namespace mmi {

// ---------------------------------------------------------------------------------------
// Dequantize: one thread per (column n, 8 consecutive k) = one MFMA B operand, computed by
// the same dequant_operand() the GEMM uses.
// ---------------------------------------------------------------------------------------
template <int FMT, class AT>
__global__ void dequant_kernel(const GemmParams p, uint16_t* __restrict__ out, int gs_mode) {
  constexpr int BITS = fmt_bits(FMT);
  const int64_t total = (int64_t)(p.K / 8) * p.N;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = idx % p.N;
    const int64_t k0 = (idx / p.N) * 8;
    const int group = gs_mode == GSM_CHANNEL ? 0 : (int)(k0 >> p.group_shift);
    const Meta m = make_meta<FMT, AT>(load_meta_raw<FMT, AT>(p, 0, group, (int)n));
    uint32_t w0, w1 = 0;
    if constexpr (BITS == 4) {
      w0 = p.b[layout_word_index(4, p.K, p.N, n, k0)];
    } else {
      w0 = p.b[layout_word_index(8, p.K, p.N, n, k0)];
      w1 = p.b[layout_word_index(8, p.K, p.N, n, k0 + 4)];
    }
    const u32x4_t v = dequant_operand<FMT, AT>(w0, w1, m, opaque_zero(p.zero));
    float alpha = 1.0f;
    if constexpr (FMT == FMT_NVFP4) alpha = __builtin_ldexpf(p.global_scale[0], p.alpha_exp);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint16_t h = (uint16_t)(v[i >> 1] >> ((i & 1) * 16));
      if constexpr (FMT == FMT_NVFP4) h = to_raw16(raw16_to_float(h, AT{}) * alpha, AT{});
      out[(k0 + i) * p.N + n] = h;
    }
  }
}

template <int FMT>
static hipError_t launch_dequant_fmt(const GemmParams& p, bool bf16, uint16_t* out, int gs_mode,
                                     hipStream_t stream) {
  const int64_t total = (int64_t)(p.K / 8) * p.N;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (bf16)
    hipLaunchKernelGGL((dequant_kernel<FMT, BF16>), dim3((unsigned)blocks), dim3(256), 0, stream, p,
                       out, gs_mode);
  else
    hipLaunchKernelGGL((dequant_kernel<FMT, F16>), dim3((unsigned)blocks), dim3(256), 0, stream, p,
                       out, gs_mode);
  return hipGetLastError();
}

hipError_t launch_dequant(int fmt, const GemmParams& p, bool bf16, void* out, int gs_mode,
                          hipStream_t stream) {
  uint16_t* o = reinterpret_cast<uint16_t*>(out);
  switch (fmt) {
    case FMT_U4B8: return launch_dequant_fmt<FMT_U4B8>(p, bf16, o, gs_mode, stream);
    case FMT_U4: return launch_dequant_fmt<FMT_U4>(p, bf16, o, gs_mode, stream);
    case FMT_U8B128: return launch_dequant_fmt<FMT_U8B128>(p, bf16, o, gs_mode, stream);
    case FMT_U8: return launch_dequant_fmt<FMT_U8>(p, bf16, o, gs_mode, stream);
    case FMT_U4Z: return launch_dequant_fmt<FMT_U4Z>(p, bf16, o, gs_mode, stream);
    case FMT_U8Z: return launch_dequant_fmt<FMT_U8Z>(p, bf16, o, gs_mode, stream);
    case FMT_FP8: return launch_dequant_fmt<FMT_FP8>(p, bf16, o, gs_mode, stream);
    case FMT_MXFP4: return launch_dequant_fmt<FMT_MXFP4>(p, bf16, o, gs_mode, stream);
    case FMT_NVFP4: return launch_dequant_fmt<FMT_NVFP4>(p, bf16, o, gs_mode, stream);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------
// Act-order activation gather (upstream gptq_marlin's permute_cols step): the weights were
// repacked with perm = argsort(g_idx), so their row j is source row perm[j]; A's columns are
// gathered the same way and the GEMM then runs on contiguous groups.  g_idx is the sorted
// one the layer passes (marlin_sort_g_idx: g_idx[perm]), so row j's group is g_idx[j], and
// the grouped kernels need it to be j / group_size: every group holds exactly group_size
// rows, as GPTQ's act-order quantizer forms them.  A column j that breaks that, or whose
// perm entry is outside [0, size_k), is written as NaN, so the result shows it without a
// host synchronisation.  Workgroup x covers 256 consecutive columns j, workgroup y walks
// rows.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void permute_cols_kernel(const uint16_t* __restrict__ a,
                                                           int64_t lda, const int* __restrict__ perm,
                                                           const int* __restrict__ g_idx,
                                                           int group_shift, int size_k, int64_t rows,
                                                           uint16_t nan_bits,
                                                           uint16_t* __restrict__ out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= size_k) return;
  const int src = perm[j];
  bool ok = src >= 0 && src < size_k;
  if (group_shift >= 0) ok = ok && g_idx[j] == (j >> group_shift);
  for (int64_t m = blockIdx.y; m < rows; m += gridDim.y)
    out[m * size_k + j] = ok ? a[m * lda + src] : nan_bits;
}

hipError_t launch_permute_cols(const void* a, bool bf16, int64_t lda, const int* perm,
                               const int* g_idx, int group_shift, int64_t size_k, int64_t size_m,
                               void* out, hipStream_t stream) {
  if (size_k == 0 || size_m == 0) return hipSuccess;
  const unsigned gx = (unsigned)((size_k + 255) / 256);
  const unsigned gy = (unsigned)std::min<int64_t>(size_m, 1024);
  hipLaunchKernelGGL(permute_cols_kernel, dim3(gx, gy), dim3(256), 0, stream,
                     reinterpret_cast<const uint16_t*>(a), lda, perm, g_idx, group_shift,
                     (int)size_k, size_m, (uint16_t)(bf16 ? 0x7fc0u : 0x7e00u),
                     reinterpret_cast<uint16_t*>(out));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Packed integer zero points -> 16-bit codes: out[e] = code e of the int32 words, where
// word e / pack holds codes e, e+1, ... from its low bits up (pack = 32 / bits).  The GEMM
// kernels then read integer zero points with the same loads as float ones.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void expand_zeros_kernel(const uint32_t* __restrict__ words,
                                                           int bits, int64_t n,
                                                           uint16_t* __restrict__ out) {
  const int pack = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x)
    out[e] = (uint16_t)((words[e / pack] >> (bits * (int)(e % pack))) & mask);
}

hipError_t launch_expand_zeros(const void* words, int bits, int64_t n_codes, void* out,
                               hipStream_t stream) {
  if (n_codes == 0) return hipSuccess;
  const unsigned grid = (unsigned)std::min<int64_t>((n_codes + 255) / 256, 16384);
  hipLaunchKernelGGL(expand_zeros_kernel, dim3(grid), dim3(256), 0, stream,
                     reinterpret_cast<const uint32_t*>(words), bits, n_codes,
                     reinterpret_cast<uint16_t*>(out));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// moe_align_block_size (reference moe_align_sum_kernels.cu:81-181, 291-320), one workgroup
// of 1024 threads; launched for more than kAlignSpreadMax routes (fewer take the
// many-workgroup kernel below, same output) and for up to 2048.  Unlike the reference's atomic scatter,
// placement is deterministic: route indices of one expert appear in ascending order.
//   * Routes are ranked in rounds of 16 x 1024 indices: wavefront w of a round takes 1024
//     consecutive indices in 16 passes of 64, ranks its lanes per expert with one ballot
//     per expert-id bit (plus the expert's count from the wavefront's earlier passes, kept
//     in LDS), and wavefronts are ordered by a per-expert prefix over the per-wave counts.
//   * Up to 16K routes (T = 2048 tokens at top-8) that one round is also the histogram: the
//     topk ids are read once, ranks stay in registers across the scan.  Larger inputs count
//     first (one LDS atomic per expert and wavefront pass), then rank and place round by
//     round.
//   * The padded prefix is a wavefront shuffle scan plus one cross-wave step.  The topk ids
//     of all 16 passes are loaded before any is inspected.
// ---------------------------------------------------------------------------------------
constexpr int kAlignPasses = 16;  // passes of 64 routes per wavefront per round

template <typename IdT>
__global__ __launch_bounds__(1024) void moe_align_kernel(
    const IdT* __restrict__ topk, int64_t numel, int E, int bs, int* __restrict__ sorted,
    int64_t sorted_numel, int* __restrict__ expert_ids, int64_t expert_ids_numel,
    int* __restrict__ post_pad, const int* __restrict__ expert_map, int has_map) {
  extern __shared__ int smem[];
  int* counts = smem;        // [E] routes per expert (whole input)
  int* cursor = counts + E;  // [E + 1] padded exclusive prefix, advanced round by round
  int* round_n = cursor + E + 1;  // [E] routes per expert in the current round
  // [16][E] per wave and expert: routes so far in this round, then the exclusive prefix over
  // the waves (both < 16 * 1024, so 16 bits suffice)
  uint16_t* wave_cnt = reinterpret_cast<uint16_t*>(round_n + E);
  __shared__ int wave_sum[16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ebits = E > 1 ? 32 - __clz(E - 1) : 1;  // bits of the largest expert id
  const uint64_t lanes_below = (1ull << lane) - 1;
  constexpr int64_t kRound = 1024 * kAlignPasses;

  // Expert of routes wbase + 64 s + lane, s < kAlignPasses (-1: none or invalid).  Every
  // pass's id is loaded before any is inspected (clamped indices, no branch between the
  // loads), then the expert_map lookups likewise, so the loads overlap.
  auto load_experts = [&](int64_t wbase, int (&ev)[kAlignPasses]) {
    const int64_t last = numel > 0 ? numel - 1 : 0;
    // passes that hold routes (wave-uniform)
    const int live = (int)max<int64_t>(0, min<int64_t>(kAlignPasses, (numel - wbase + 63) / 64));
    int64_t raw[kAlignPasses];
#pragma unroll
    for (int s = 0; s < kAlignPasses; ++s)
      raw[s] = s < live ? (int64_t)topk[min(wbase + s * 64 + lane, last)] : -1;
#pragma unroll
    for (int s = 0; s < kAlignPasses; ++s) {
      const bool ok = wbase + s * 64 + lane < numel && raw[s] >= 0 && raw[s] < E;
      ev[s] = ok ? (int)raw[s] : -1;
    }
    if (has_map) {
      int me[kAlignPasses];
#pragma unroll
      for (int s = 0; s < kAlignPasses; ++s) me[s] = expert_map[ev[s] >= 0 ? ev[s] : 0];
#pragma unroll
      for (int s = 0; s < kAlignPasses; ++s)
        ev[s] = (ev[s] >= 0 && me[s] >= 0 && me[s] < E) ? me[s] : -1;
    }
  };
  // lanes of this wave holding the same expert as this lane: intersect, over the id's bits,
  // the ballots that agree with this lane's bit (no per-expert loop)
  auto same_expert = [&](int e) -> uint64_t {
    uint64_t same = __ballot(e >= 0);
    for (int bit = 0; bit < ebits; ++bit) {
      const int set = (e >> bit) & 1;
      const uint64_t m = __ballot(set);
      same &= set ? m : ~m;
    }
    return same;
  };

  // Rank the round starting at `base`: ex / rk get each pass's expert and its rank among
  // the wave's routes of that expert; then wave_cnt holds the wave-exclusive prefix and
  // round_n the round's count per expert.
  int ex[kAlignPasses], rk[kAlignPasses];
  auto rank_round = [&](int64_t base) {
    const int64_t wbase = base + (int64_t)wave * 64 * kAlignPasses;
    for (int x = lane; x < E; x += 64) wave_cnt[wave * E + x] = 0;  // this wave's row only
    load_experts(wbase, ex);
#pragma unroll
    for (int s = 0; s < kAlignPasses; ++s) {
      rk[s] = 0;
      if (wbase + s * 64 >= numel) continue;  // wave-uniform: passes past the end
      const int e = ex[s];
      const uint64_t same = same_expert(e);
      const uint64_t before = same & lanes_below;
      int r = 0;
      if (e >= 0) r = wave_cnt[wave * E + e] + __popcll(before);
      // the leader's store depends on its own read, so every lane of the wave has read the
      // old count before it lands
      if (e >= 0 && before == 0) wave_cnt[wave * E + e] = (uint16_t)(r + __popcll(same));
      rk[s] = r;
    }
    __syncthreads();
    if (numel - base <= 64 * kAlignPasses) {
      // every route of the round is in wavefront 0 (the others' rows are zero): its counts
      // are the round's, its exclusive prefix is zero
      for (int x = tid; x < E; x += 1024) {
        round_n[x] = wave_cnt[x];
        wave_cnt[x] = 0;
      }
    } else {
      for (int x = tid; x < E; x += 1024) {
        int run = 0;
        for (int w = 0; w < 16; ++w) {
          const int c = wave_cnt[w * E + x];
          wave_cnt[w * E + x] = (uint16_t)run;
          run += c;
        }
        round_n[x] = run;
      }
    }
    __syncthreads();
  };
  auto place_round = [&](int64_t base) {
    const int64_t wbase = base + (int64_t)wave * 64 * kAlignPasses;
#pragma unroll
    for (int s = 0; s < kAlignPasses; ++s) {
      const int e = ex[s];
      if (e >= 0) {
        const int pos = cursor[e] + wave_cnt[wave * E + e] + rk[s];
        if (pos < sorted_numel) sorted[pos] = (int)(wbase + s * 64 + lane);
      }
    }
  };

  // sentinels everywhere first (coalesced; placement overwrites the route slots after the
  // barriers below, which also wait for these stores)
  for (int64_t j = tid; j < sorted_numel; j += 1024) sorted[j] = (int)numel;

  const bool one_round = numel <= kRound;
  if (one_round) {
    rank_round(0);
    for (int x = tid; x < E; x += 1024) counts[x] = round_n[x];
  } else {
    for (int x = tid; x < E; x += 1024) counts[x] = 0;
    __syncthreads();
    for (int64_t base = 0; base < numel; base += kRound) {
      const int64_t wbase = base + (int64_t)wave * 64 * kAlignPasses;
      int ev[kAlignPasses];
      load_experts(wbase, ev);
#pragma unroll
      for (int s = 0; s < kAlignPasses; ++s) {
        if (wbase + s * 64 >= numel) continue;
        const uint64_t same = same_expert(ev[s]);
        if (ev[s] >= 0 && (same & lanes_below) == 0) atomicAdd(&counts[ev[s]], __popcll(same));
      }
    }
  }
  __syncthreads();

  // padded exclusive prefix (E <= 1024: one expert per thread)
  const int pad = tid < E ? (counts[tid] + bs - 1) / bs * bs : 0;
  int incl = pad;
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) wave_sum[wave] = incl;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < 16; ++w) incl += w < wave ? wave_sum[w] : 0;
  const int start = incl - pad;
  if (tid < E) cursor[tid] = start;
  if (tid == E - 1) cursor[E] = incl;
  __syncthreads();
  const int total = cursor[E];
  if (tid == 0) post_pad[0] = total;

  // expert_ids
  if (tid < E) {
    for (int b = start / bs; b < incl / bs; ++b)
      if (b < expert_ids_numel) expert_ids[b] = tid;
  }
  for (int64_t b = total / bs + tid; b < expert_ids_numel; b += 1024) expert_ids[b] = -1;

  if (one_round) {
    place_round(0);
    return;
  }
  for (int64_t base = 0; base < numel; base += kRound) {
    rank_round(base);
    place_round(base);
    __syncthreads();
    for (int x = tid; x < E; x += 1024) cursor[x] += round_n[x];
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------
// Many-workgroup moe_align_block_size, for 2049 to kAlignSpreadMax routes (the placement is
// the same stable order as above).  Workgroup g ranks routes [1024 g, 1024 g + 1024), one
// 64-route pass per wavefront.  Each workgroup first histograms every route in LDS -- the
// totals per expert and the counts of the chunks before its own -- so no workgroup waits for
// another, and the padded prefix is computed redundantly in each.  Workgroup 0 alone writes
// num_tokens_post_pad, expert_ids and the sentinels, which fill only padding slots (those
// of each expert after its routes, and those past the padded total): no slot is written by
// two workgroups.
// ---------------------------------------------------------------------------------------
constexpr int64_t kAlignSpreadMax = 65536;

template <typename IdT>
__global__ __launch_bounds__(1024) void moe_align_spread_kernel(
    const IdT* __restrict__ topk, int64_t numel, int E, int bs, int* __restrict__ sorted,
    int64_t sorted_numel, int* __restrict__ expert_ids, int64_t expert_ids_numel,
    int* __restrict__ post_pad, const int* __restrict__ expert_map, int has_map) {
  extern __shared__ int smem[];
  int* rest = smem;               // [E] routes per expert from this chunk on
  int* before = rest + E;         // [E] routes per expert in the chunks before this one
  int* start = before + E;        // [E + 1] padded exclusive prefix
  uint16_t* wave_cnt = reinterpret_cast<uint16_t*>(start + E + 1);  // [16][E]
  __shared__ int wave_sum[16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ebits = E > 1 ? 32 - __clz(E - 1) : 1;
  const int64_t chunk0 = (int64_t)blockIdx.x * 1024;

  // expert of route i (-1: out of range, invalid or unmapped), as moe_align_kernel
  auto expert_of = [&](int64_t i) -> int {
    if (i >= numel) return -1;
    const int64_t raw = (int64_t)topk[i];
    int e = (raw >= 0 && raw < E) ? (int)raw : -1;
    if (has_map && e >= 0) {
      const int m = expert_map[e];
      e = (m >= 0 && m < E) ? m : -1;
    }
    return e;
  };

  for (int x = tid; x < E; x += 1024) rest[x] = 0, before[x] = 0;
  for (int x = lane; x < E; x += 64) wave_cnt[wave * E + x] = 0;  // this wave's row
  // this workgroup's route and its rank among the wave's routes of the same expert
  const int64_t mine = chunk0 + wave * 64 + lane;
  const int em = expert_of(mine);
  uint64_t same = __ballot(em >= 0);
  for (int bit = 0; bit < ebits; ++bit) {
    const int set = (em >> bit) & 1;
    const uint64_t m = __ballot(set);
    same &= set ? m : ~m;
  }
  const uint64_t below = same & ((1ull << lane) - 1);
  const int rank = __popcll(below);
  // the leader of each expert in the wave records the wave's count (after this wave's
  // zeroing above: one wavefront's LDS accesses stay in program order)
  if (em >= 0 && below == 0) wave_cnt[wave * E + em] = (uint16_t)__popcll(same);
  __syncthreads();

  // histogram of every route, 8 loads in flight per thread
  constexpr int kLoads = 8;
  for (int64_t base = 0; base < numel; base += 1024 * kLoads) {
    int ev[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) ev[j] = expert_of(base + j * 1024 + tid);
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      if (ev[j] >= 0) atomicAdd(base + j * 1024 + tid < chunk0 ? &before[ev[j]] : &rest[ev[j]], 1);
  }
  // per expert: exclusive prefix of the wave counts over this workgroup's waves
  for (int x = tid; x < E; x += 1024) {
    int run = 0;
    for (int w = 0; w < 16; ++w) {
      const int c = wave_cnt[w * E + x];
      wave_cnt[w * E + x] = (uint16_t)run;
      run += c;
    }
  }
  __syncthreads();

  // padded exclusive prefix (E <= 1024: one expert per thread)
  const int cnt = tid < E ? before[tid] + rest[tid] : 0;
  const int pad = (cnt + bs - 1) / bs * bs;
  int incl = pad;
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) wave_sum[wave] = incl;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < 16; ++w) incl += w < wave ? wave_sum[w] : 0;
  const int first = incl - pad;
  if (tid < E) start[tid] = first;
  if (tid == E - 1) start[E] = incl;
  __syncthreads();

  if (em >= 0) {
    const int64_t pos = (int64_t)start[em] + before[em] + wave_cnt[wave * E + em] + rank;
    if (pos < sorted_numel) sorted[pos] = (int)mine;
  }
  if (blockIdx.x != 0) return;
  const int padded_total = start[E];
  if (tid == 0) post_pad[0] = padded_total;
  if (tid < E) {
    for (int64_t j = first + cnt; j < incl && j < sorted_numel; ++j) sorted[j] = (int)numel;
    for (int b = first / bs; b < incl / bs; ++b)
      if (b < expert_ids_numel) expert_ids[b] = tid;
  }
  for (int64_t j = padded_total + tid; j < sorted_numel; j += 1024) sorted[j] = (int)numel;
  for (int64_t b = padded_total / bs + tid; b < expert_ids_numel; b += 1024) expert_ids[b] = -1;
}

hipError_t launch_moe_align(const void* topk, bool is64, int64_t numel, int E, int bs, int* sorted,
                            int64_t sorted_numel, int* expert_ids, int64_t expert_ids_numel,
                            int* post_pad, const int* expert_map, hipStream_t stream) {
  const size_t smem = (size_t)(3 * E + 1) * sizeof(int) + (size_t)16 * E * sizeof(uint16_t);
  // (up to two chunks the single workgroup is as fast: 6.2 against 7.8 us at 128 routes)
  if (numel > 2048 && numel <= kAlignSpreadMax) {
    const unsigned grid = (unsigned)std::max<int64_t>(1, (numel + 1023) / 1024);
    if (is64)
      hipLaunchKernelGGL((moe_align_spread_kernel<int64_t>), dim3(grid), dim3(1024), smem, stream,
                         reinterpret_cast<const int64_t*>(topk), numel, E, bs, sorted,
                         sorted_numel, expert_ids, expert_ids_numel, post_pad, expert_map,
                         expert_map ? 1 : 0);
    else
      hipLaunchKernelGGL((moe_align_spread_kernel<int32_t>), dim3(grid), dim3(1024), smem, stream,
                         reinterpret_cast<const int32_t*>(topk), numel, E, bs, sorted,
                         sorted_numel, expert_ids, expert_ids_numel, post_pad, expert_map,
                         expert_map ? 1 : 0);
    return hipGetLastError();
  }
  if (is64)
    hipLaunchKernelGGL((moe_align_kernel<int64_t>), dim3(1), dim3(1024), smem, stream,
                       reinterpret_cast<const int64_t*>(topk), numel, E, bs, sorted, sorted_numel,
                       expert_ids, expert_ids_numel, post_pad, expert_map, expert_map ? 1 : 0);
  else
    hipLaunchKernelGGL((moe_align_kernel<int32_t>), dim3(1), dim3(1024), smem, stream,
                       reinterpret_cast<const int32_t*>(topk), numel, E, bs, sorted, sorted_numel,
                       expert_ids, expert_ids_numel, post_pad, expert_map, expert_map ? 1 : 0);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// moe_sum: out[t, h] = sum_k in[t, k, h] as the reference computes it
// (moe_align_sum_kernels.cu:350-363, 597-639): for top-k 2..4 its kernel adds in the element
// type, rounding after every addition; otherwise at::sum_out accumulates in fp32 and rounds
// once.  `step_round` selects the former.  fp32 inputs add in fp32 either way (for top-k
// beyond 4 in index order; at::sum_out's order is its own, so fp32 agrees to rounding).
// ---------------------------------------------------------------------------------------
template <class AT>
__device__ __forceinline__ float moe_sum_add(float s, float x, bool step_round) {
  const float v = s + x;
  return step_round ? raw16_to_float(to_raw16(v, AT{}), AT{}) : v;
}

// One output element per thread, any hidden size and alignment; the flat index runs over
// tokens x hidden, so the token count is not limited by a grid dimension.
template <class AT>
__global__ void moe_sum_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                               int64_t tokens, int topk, int64_t hidden) {
  const bool step_round = topk >= 2 && topk <= 4;
  const int64_t n = tokens * hidden;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / hidden;
    const int64_t h = i - t * hidden;
    float s = 0.f;
    for (int k = 0; k < topk; ++k)
      s = moe_sum_add<AT>(s, raw16_to_float(in[(t * topk + k) * hidden + h], AT{}), step_round);
    out[i] = to_raw16(s, AT{});
  }
}

__global__ void moe_sum_kernel_f32(const float* __restrict__ in, float* __restrict__ out,
                                   int64_t tokens, int topk, int64_t hidden) {
  const int64_t n = tokens * hidden;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / hidden;
    const int64_t h = i - t * hidden;
    float s = 0.f;
    for (int k = 0; k < topk; ++k) s += in[(t * topk + k) * hidden + h];
    out[i] = s;
  }
}

// hidden % 8 == 0 and 16-byte aligned rows: 8 outputs per thread, each top-k slice read
// with one 16-byte load, four slices in flight; same arithmetic as above.
template <class AT>
__global__ void moe_sum_kernel_v8(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                  int64_t tokens, int topk, int64_t hidden) {
  const int64_t per_row = hidden >> 3;
  const int64_t n = tokens * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_row;
    const int64_t h = (i - t * per_row) << 3;
    const uint16_t* src = in + t * topk * hidden + h;
    const bool step_round = topk >= 2 && topk <= 4;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < topk; k0 += 4) {
      u32x4_t v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (k0 + j < topk) v[j] = *reinterpret_cast<const u32x4_t*>(src + (int64_t)(k0 + j) * hidden);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (k0 + j < topk) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            s[2 * w] = moe_sum_add<AT>(s[2 * w], raw16_to_float(v[j][w] & 0xffffu, AT{}), step_round);
            s[2 * w + 1] = moe_sum_add<AT>(s[2 * w + 1], raw16_to_float(v[j][w] >> 16, AT{}), step_round);
          }
        }
      }
    }
    u32x4_t o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = pack2(s[2 * w], s[2 * w + 1], AT{});
    *reinterpret_cast<u32x4_t*>(out + t * hidden + h) = o;
  }
}

// kind: 0 fp16, 1 bf16, 2 fp32
hipError_t launch_moe_sum(const void* in, int kind, int64_t tokens, int topk, int64_t hidden,
                          void* out, hipStream_t stream) {
  if (tokens == 0 || hidden == 0) return hipSuccess;
  const int64_t total = tokens * hidden;
  if (kind == 2) {
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 256 * 16);
    hipLaunchKernelGGL(moe_sum_kernel_f32, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<const float*>(in), reinterpret_cast<float*>(out), tokens,
                       topk, hidden);
    return hipGetLastError();
  }
  const bool bf16 = kind == 1;
  const uint16_t* i16 = reinterpret_cast<const uint16_t*>(in);
  uint16_t* o16 = reinterpret_cast<uint16_t*>(out);
  if (hidden % 8 == 0 && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    const int64_t n = tokens * (hidden / 8);
    const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 256 * 16);
    if (bf16)
      hipLaunchKernelGGL((moe_sum_kernel_v8<BF16>), dim3(blocks), dim3(256), 0, stream, i16, o16,
                         tokens, topk, hidden);
    else
      hipLaunchKernelGGL((moe_sum_kernel_v8<F16>), dim3(blocks), dim3(256), 0, stream, i16, o16,
                         tokens, topk, hidden);
    return hipGetLastError();
  }
  const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 256 * 16);
  if (bf16)
    hipLaunchKernelGGL((moe_sum_kernel<BF16>), dim3(blocks), dim3(256), 0, stream, i16, o16,
                       tokens, topk, hidden);
  else
    hipLaunchKernelGGL((moe_sum_kernel<F16>), dim3(blocks), dim3(256), 0, stream, i16, o16,
                       tokens, topk, hidden);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// silu_and_mul: out[r, j] = silu(x[r, j]) * x[r, d + j], rounded as the reference's torch
// expression F.silu(gate) * up rounds: silu to the element type, then the product.
// ---------------------------------------------------------------------------------------

// d % 8 == 0: 8 outputs (16 bytes) per thread
template <class AT>
__global__ void silu_mul_kernel_v8(const uint16_t* __restrict__ x, uint16_t* __restrict__ out,
                                   int64_t rows, int64_t d) {
  const int64_t per_row = d >> 3;
  const int64_t n = rows * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row;
    const int64_t c = (i - r * per_row) * 8;
    const u32x4_t g = *reinterpret_cast<const u32x4_t*>(x + r * 2 * d + c);
    const u32x4_t u = *reinterpret_cast<const u32x4_t*>(x + r * 2 * d + d + c);
    u32x4_t o;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      o[w] = pack2(silu_mul1<AT>(g[w], u[w]), silu_mul1<AT>(g[w] >> 16, u[w] >> 16), AT{});
    *reinterpret_cast<u32x4_t*>(out + r * d + c) = o;
  }
}

template <class AT>
__global__ void silu_mul_kernel_v1(const uint16_t* __restrict__ x, uint16_t* __restrict__ out,
                                   int64_t rows, int64_t d) {
  const int64_t n = rows * d;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / d;
    const int64_t c = i - r * d;
    out[i] = to_raw16(silu_mul1<AT>(x[r * 2 * d + c], x[r * 2 * d + d + c]), AT{});
  }
}

hipError_t launch_silu_and_mul(const void* x, bool bf16, int64_t rows, int64_t d, void* out,
                               hipStream_t stream) {
  if (rows == 0 || d == 0) return hipSuccess;
  const uint16_t* x16 = reinterpret_cast<const uint16_t*>(x);
  uint16_t* o16 = reinterpret_cast<uint16_t*>(out);
  const bool v8 = d % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const int64_t work = v8 ? rows * (d / 8) : rows * d;
  const unsigned grid = (unsigned)std::min<int64_t>((work + 255) / 256, 8192);
  if (v8) {
    if (bf16) hipLaunchKernelGGL((silu_mul_kernel_v8<BF16>), dim3(grid), dim3(256), 0, stream, x16, o16, rows, d);
    else hipLaunchKernelGGL((silu_mul_kernel_v8<F16>), dim3(grid), dim3(256), 0, stream, x16, o16, rows, d);
  } else {
    if (bf16) hipLaunchKernelGGL((silu_mul_kernel_v1<BF16>), dim3(grid), dim3(256), 0, stream, x16, o16, rows, d);
    else hipLaunchKernelGGL((silu_mul_kernel_v1<F16>), dim3(grid), dim3(256), 0, stream, x16, o16, rows, d);
  }
  return hipGetLastError();
}

}  // namespace mmi
