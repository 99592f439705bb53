// router_kernels.hip -- MoE router: topk_softmax / topk_sigmoid.
//
// Semantics (reference csrc/moe/topk_softmax_kernels.cu): per token row, scores are the fp32
// softmax over the experts (:75-133) or the elementwise sigmoid (:135-153); experts are chosen
// by score + bias (bias optional, fp32 [E]) in descending order, ties going to the lower
// expert index (:488, :508); the returned weight is the unbiased score (:223-225), divided by
// the sum of the k chosen scores when renormalize is set (a zero sum divides by 1, :551-560);
// token_expert_indices[t, j] = j * num_tokens + t (:226, :527).
//
// Layout on MI355X: one 64-lane wavefront per token.  Lane l holds experts l + 64*j for
// j < VPL in registers, so each j is one coalesced 64-element load of the row; the softmax
// max / sum are reductions across the wave in VALU cross-lane operations (DPP, permlane
// swaps), and the top k are chosen by a threshold search over ballots (choose_topk) instead
// of k dependent argmax rounds.  No workspace: the reference's E > 256 / non-power-of-two path goes through a
// [T, E] fp32 workspace (:774-777); here every E <= 64 * 64 stays in registers.
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "host_common.h"

namespace mmi {

namespace {

template <class IT>
struct ScoreIn;
template <>
struct ScoreIn<float> {
  using raw = float;
  __device__ static float get(const float* p, int64_t i) { return p[i]; }
};
template <>
struct ScoreIn<F16> {
  using raw = uint16_t;
  __device__ static float get(const uint16_t* p, int64_t i) { return raw16_to_float(p[i], F16{}); }
};
template <>
struct ScoreIn<BF16> {
  using raw = uint16_t;
  __device__ static float get(const uint16_t* p, int64_t i) {
    return raw16_to_float(p[i], BF16{});
  }
};

// Cross-lane reductions without LDS round trips: DPP inside each 16-lane row (row_ror:8,
// row_ror:4, then quad xor 2 and xor 1), then v_permlane16_swap / v_permlane32_swap across
// rows.  permlane{16,32}_swap(v, v) returns the lane's own row value and its partner row's
// value (in row order), so combining the pair with a commutative operation gives every lane
// the same result.  In this order every lane also forms the same association of partial
// results, so a float sum is bit-identical on all 64 lanes.
constexpr int kDppRor8 = 0x128;
constexpr int kDppRor4 = 0x124;
constexpr int kDppXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kDppXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(int, v)));
}

// The two values of a row pair (16-lane rows 2r, 2r+1) or half pair (lanes 0-31, 32-63).
struct Pair {
  float v0, v1;
};
__device__ __forceinline__ Pair swap16(float v) {
  const int b = __builtin_bit_cast(int, v);
  const auto sv = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  return {__builtin_bit_cast(float, (int)sv[0]), __builtin_bit_cast(float, (int)sv[1])};
}
__device__ __forceinline__ Pair swap32(float v) {
  const int b = __builtin_bit_cast(int, v);
  const auto sv = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return {__builtin_bit_cast(float, (int)sv[0]), __builtin_bit_cast(float, (int)sv[1])};
}

// Merges two (largest, second largest) pairs of a multiset: a repeated maximum counts twice.
__device__ __forceinline__ void top2_merge(float a1, float b1, float a2, float b2, float& m1,
                                           float& m2) {
  m1 = fmaxf(a1, b1);
  m2 = fmaxf(fminf(a1, b1), fmaxf(a2, b2));
}
template <int CTRL>
__device__ __forceinline__ void top2_dpp(float& m1, float& m2) {
  const float o1 = dpp<CTRL>(m1), o2 = dpp<CTRL>(m2);
  top2_merge(m1, o1, m2, o2, m1, m2);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppRor8>(v));
  v = fmaxf(v, dpp<kDppRor4>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppXor1>(v));
  Pair p = swap16(v);
  v = fmaxf(p.v0, p.v1);
  p = swap32(v);
  return fmaxf(p.v0, p.v1);
}

__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp<kDppRor8>(v);
  v = v + dpp<kDppRor4>(v);
  v = v + dpp<kDppXor2>(v);
  v = v + dpp<kDppXor1>(v);
  Pair p = swap16(v);
  v = p.v0 + p.v1;
  p = swap32(v);
  return p.v0 + p.v1;
}

constexpr int kSoftmax = 0;  // topk_gating scoring
constexpr int kScoreNone = 0;  // grouped_topk scoring_func 0: the scores as given
constexpr int kSigmoid = 1;
constexpr int kWavesPerBlock = 4;

// Order-preserving key of a float (a larger float gives a larger unsigned key; -0 and +0 share
// one key, as they compare equal).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// One wave's chosen experts, in expert order, before ranking.
struct ChosenList {
  uint32_t key[kMaxK];
  int idx[kMaxK];
  float w[kMaxK];
};

// Chooses the k largest keys among the live slots of the wave (slot j of lane l is expert
// l + 64*j; equal keys go to the lower expert) without k dependent argmax rounds:
//  1. a threshold tau with at least k live keys >= tau and fewer than k above it, found bit
//     by bit from the top (each step one compare per slot and a ballot count; the search
//     stops once exactly k keys are >= tau);
//  2. every key above tau, then the lowest-expert keys equal to tau until k are chosen;
//  3. the chosen (key, expert, w) are compacted into `out` in expert order.
// Returns the sum of the chosen w, the same on every lane.
template <int VPL>
__device__ __forceinline__ float choose_topk(const uint32_t (&key)[VPL], const float (&w)[VPL],
                                             uint64_t live, int k, int lane, ChosenList& out) {
  uint32_t tau = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) cnt += __popcll(__ballot(((live >> j) & 1) && key[j] >= cand));
    if (cnt >= k) {
      tau = cand;
      if (cnt == k) break;  // exactly k keys >= tau: a larger tau would choose the same set
    }
  }
  int above = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) above += __popcll(__ballot(((live >> j) & 1) && key[j] > tau));
  const int need = k - above;  // keys equal to tau still to take, lowest experts first
  int eq_before = 0;
  int base = 0;
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const bool lv = (live >> j) & 1;
    const uint64_t eq = __ballot(lv && key[j] == tau);
    const bool take = lv && (key[j] > tau || (key[j] == tau && eq_before + lanes_below(eq) < need));
    eq_before += __popcll(eq);
    const uint64_t tm = __ballot(take);
    if (take) {
      const int pos = base + lanes_below(tm);
      out.key[pos] = key[j];
      out.idx[pos] = lane + 64 * j;
      out.w[pos] = w[j];
      sum += w[j];
    }
    base += __popcll(tm);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return wave_sum(sum);
}

// Calls store(rank, expert, w) for each of the k chosen entries, rank = its place in
// descending key order (ties: the lower expert, which is the earlier list entry).
template <class F>
__device__ __forceinline__ void emit_ranked(const ChosenList& c, int k, int lane, F&& store) {
  for (int r = lane; r < k; r += 64) {
    const uint32_t kr = c.key[r];
    int rank = 0;
    for (int q = 0; q < k; ++q) {
      const uint32_t kq = c.key[q];
      rank += (kq > kr || (kq == kr && q < r)) ? 1 : 0;
    }
    store(rank, c.idx[r], c.w[r]);
  }
}

// VPL: experts per lane (E <= 64 * VPL).  OT: id output type (int32_t, uint32_t, int64_t).
template <class IT, int VPL, int SF, class OT>
__global__ __launch_bounds__(64 * kWavesPerBlock) void topk_gating_kernel(
    const typename ScoreIn<IT>::raw* __restrict__ gating, const float* __restrict__ bias,
    float* __restrict__ weights, OT* __restrict__ ids, int* __restrict__ token_expert_indices,
    int64_t num_tokens, int num_experts, int k, int renormalize) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (t >= num_tokens) return;  // whole wave leaves together; no barriers below
  const typename ScoreIn<IT>::raw* row = gating + t * num_experts;

  float score[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    score[j] = e < num_experts ? ScoreIn<IT>::get(row, e) : -INFINITY;
  }

  if constexpr (SF == kSoftmax) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j) m = fmaxf(m, score[j]);
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = lane + 64 * j;
      score[j] = e < num_experts ? expf(score[j] - m) : 0.0f;
      s += score[j];
    }
    const float inv = 1.0f / wave_sum(s);
#pragma unroll
    for (int j = 0; j < VPL; ++j) score[j] *= inv;
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) score[j] = 1.0f / (1.0f + expf(-score[j]));
  }

  uint64_t live = 0;  // bit j: expert lane + 64*j exists
  uint32_t key[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    if (e < num_experts) live |= 1ull << j;
    key[j] = order_key(e < num_experts && bias ? score[j] + bias[e] : score[j]);
  }
  __shared__ ChosenList chosen[kWavesPerBlock];
  ChosenList& c = chosen[threadIdx.x >> 6];
  const float sum = choose_topk<VPL>(key, score, live, k, lane, c);
  const float denom = renormalize ? (sum > 0.0f ? sum : 1.0f) : 1.0f;
  float* wrow = weights + t * k;
  OT* irow = ids + t * k;
  int* srow = token_expert_indices + t * k;
  emit_ranked(c, k, lane, [&](int rank, int e, float w) {
    irow[rank] = (OT)e;
    wrow[rank] = renormalize ? w / denom : w;
  });
  for (int r = lane; r < k; r += 64) srow[r] = (int)((int64_t)r * num_tokens + t);
}

// ---------------------------------------------------------------------------------------
// grouped_topk (reference csrc/moe/grouped_topk_kernels.cu:517-657, host :987-1090): the
// experts form n_group equal groups; a group's score is the sum of its two largest
// score + bias values (:469-512); the topk_group best groups are kept (ties to the lower
// group, :576-585; here by counting, per group lane, the groups that beat it); the top-k experts of the kept groups by score + bias follow (ties to the
// lower expert); weights are the unbiased scores times routed_scaling_factor, divided by
// (1e-20 + their sum) when renormalizing (:639-656).  If the last kept group's score is -inf
// the row falls back to experts 0..k-1 with weight 1/k (:587-600).  Inputs that are not
// finite do not compete (their choice is -inf, :623-628).
// Scores are computed in fp32 (the reference test oracle's arithmetic,
// tests/test_marlin_moe.py:136-191).  Groups of 16, 32 or 64 experts take their top two by
// cross-lane steps; other sizes pass the choices through LDS so that lane g scans group g.
// ---------------------------------------------------------------------------------------
template <class BT>
__device__ __forceinline__ float load_bias(const void* b, int e) {
  if constexpr (std::is_same<BT, float>::value) return reinterpret_cast<const float*>(b)[e];
  else return raw16_to_float(reinterpret_cast<const uint16_t*>(b)[e], BT{});
}

template <class IT, class BT, int VPL, int SF>
__global__ __launch_bounds__(64 * kWavesPerBlock) void grouped_topk_kernel(
    const typename ScoreIn<IT>::raw* __restrict__ scores_in, const void* __restrict__ bias,
    float* __restrict__ values, int* __restrict__ ids, int64_t num_tokens, int num_experts,
    int n_group, int topk_group, int k, int renormalize, float routed_scaling_factor) {
  __shared__ float choice_lds[kWavesPerBlock][kGroupedMaxExperts];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  if (t >= num_tokens) return;  // whole wave; LDS is per wave, no barriers below
  const typename ScoreIn<IT>::raw* row = scores_in + t * num_experts;
  const int epg = num_experts / n_group;

  float score[VPL];
  float choice[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    float x = e < num_experts ? ScoreIn<IT>::get(row, e) : 0.0f;
    const bool finite = e < num_experts && __builtin_isfinite(x);
    if constexpr (SF == kSigmoid) x = 1.0f / (1.0f + expf(-x));
    score[j] = x;
    choice[j] = finite ? x + load_bias<BT>(bias, e) : -INFINITY;
  }

  // group scores (the sum of each group's two largest choices) into gscore_lds[wave][g]
  __shared__ float gscore_lds[kWavesPerBlock][32];
  if (epg == 16 || epg == 32 || epg == 64) {
    // a group is one 16-lane row, a row pair or the whole wave of a slot: merge (largest,
    // second largest) pairs with the cross-lane steps; the group's first lane writes it
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float m1 = choice[j], m2 = -INFINITY;
      top2_dpp<kDppRor8>(m1, m2);
      top2_dpp<kDppRor4>(m1, m2);
      top2_dpp<kDppXor2>(m1, m2);
      top2_dpp<kDppXor1>(m1, m2);
      if (epg >= 32) {
        const Pair a = swap16(m1), b = swap16(m2);
        top2_merge(a.v0, a.v1, b.v0, b.v1, m1, m2);  // the rows' largest, then seconds
      }
      if (epg == 64) {
        const Pair a = swap32(m1), b = swap32(m2);
        top2_merge(a.v0, a.v1, b.v0, b.v1, m1, m2);  // the rows' largest, then seconds
      }
      const int e = lane + 64 * j;
      if (e < num_experts && e % epg == 0) gscore_lds[wave][e / epg] = m1 + m2;
    }
  } else {
    // other group sizes: lane g < n_group scans group g through LDS
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = lane + 64 * j;
      if (e < num_experts) choice_lds[wave][e] = choice[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < n_group) {
      float m1 = -INFINITY, m2 = -INFINITY;
      const float* grp = &choice_lds[wave][lane * epg];
      for (int i = 0; i < epg; ++i) {
        const float v = grp[i];
        if (v > m1) {
          m2 = m1;
          m1 = v;
        } else if (v > m2) {
          m2 = v;
        }
      }
      gscore_lds[wave][lane] = epg >= 2 ? m1 + m2 : m1;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float gscore = lane < n_group ? gscore_lds[wave][lane] : -INFINITY;

  // keep the topk_group best groups: lane g counts the groups that beat it (a larger score,
  // or an equal score and a lower index) and is kept when fewer than topk_group do
  int rank = 64;
  if (lane < n_group) {
    rank = 0;
    for (int h = 0; h < n_group; ++h) {
      const float o = gscore_lds[wave][h];
      rank += (o > gscore || (o == gscore && h < lane)) ? 1 : 0;
    }
  }
  const uint32_t kept = (uint32_t)__ballot(rank < topk_group);  // wave-uniform group mask
  // the last kept group scores -inf exactly when fewer than topk_group groups score above -inf
  const int finite_groups = __popcll(__ballot(lane < n_group && gscore > -INFINITY));
  float* vrow = values + t * k;
  int* irow = ids + t * k;
  if (finite_groups < topk_group) {
    for (int r = lane; r < k; r += 64) {
      irow[r] = r;
      vrow[r] = 1.0f / (float)k;
    }
    return;
  }

  uint64_t live = 0;  // bit j: expert lane + 64*j exists and sits in a kept group
  uint32_t key[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    if (e < num_experts && ((kept >> (e / epg)) & 1)) live |= 1ull << j;
    key[j] = order_key(choice[j]);
  }
  __shared__ ChosenList chosen[kWavesPerBlock];
  const float sum = choose_topk<VPL>(key, score, live, k, lane, chosen[wave]);
  const float scale =
      renormalize ? routed_scaling_factor / (1e-20f + sum) : routed_scaling_factor;
  emit_ranked(chosen[wave], k, lane, [&](int rank, int e, float w) {
    irow[rank] = e;
    vrow[rank] = w * scale;
  });
}

template <class IT, class BT, int SF>
hipError_t launch_grouped_vpl(const void* scores, const void* bias, float* values, int* ids,
                              int64_t T, int E, int n_group, int topk_group, int k, bool renorm,
                              float rsf, hipStream_t stream) {
  const dim3 grid((unsigned)((T + kWavesPerBlock - 1) / kWavesPerBlock));
  const dim3 block(64 * kWavesPerBlock);
  using R = typename ScoreIn<IT>::raw;
  const R* g = reinterpret_cast<const R*>(scores);
#define MMI_GROUPED_LAUNCH(V)                                                                 \
  hipLaunchKernelGGL((grouped_topk_kernel<IT, BT, V, SF>), grid, block, 0, stream, g, bias,   \
                     values, ids, T, E, n_group, topk_group, k, (int)renorm, rsf)
  const int vpl = (E + 63) / 64;
  if (vpl <= 1) MMI_GROUPED_LAUNCH(1);
  else if (vpl <= 2) MMI_GROUPED_LAUNCH(2);
  else if (vpl <= 4) MMI_GROUPED_LAUNCH(4);
  else if (vpl <= 8) MMI_GROUPED_LAUNCH(8);
  else MMI_GROUPED_LAUNCH(16);
#undef MMI_GROUPED_LAUNCH
  return hipGetLastError();
}

template <class IT, int SF>
hipError_t launch_grouped_bias(int bias_kind, const void* scores, const void* bias,
                               float* values, int* ids, int64_t T, int E, int n_group,
                               int topk_group, int k, bool renorm, float rsf,
                               hipStream_t stream) {
  switch (bias_kind) {
    case 0: return launch_grouped_vpl<IT, F16, SF>(scores, bias, values, ids, T, E, n_group, topk_group, k, renorm, rsf, stream);
    case 1: return launch_grouped_vpl<IT, BF16, SF>(scores, bias, values, ids, T, E, n_group, topk_group, k, renorm, rsf, stream);
    default: return launch_grouped_vpl<IT, float, SF>(scores, bias, values, ids, T, E, n_group, topk_group, k, renorm, rsf, stream);
  }
}

template <int SF>
hipError_t launch_grouped_in(int in_kind, int bias_kind, const void* scores, const void* bias,
                             float* values, int* ids, int64_t T, int E, int n_group,
                             int topk_group, int k, bool renorm, float rsf, hipStream_t stream) {
  switch (in_kind) {
    case 0: return launch_grouped_bias<F16, SF>(bias_kind, scores, bias, values, ids, T, E, n_group, topk_group, k, renorm, rsf, stream);
    case 1: return launch_grouped_bias<BF16, SF>(bias_kind, scores, bias, values, ids, T, E, n_group, topk_group, k, renorm, rsf, stream);
    default: return launch_grouped_bias<float, SF>(bias_kind, scores, bias, values, ids, T, E, n_group, topk_group, k, renorm, rsf, stream);
  }
}

template <class IT, int SF, class OT>
hipError_t launch_vpl(const void* gating, const float* bias, float* w, OT* ids, int* tei,
                      int64_t T, int E, int k, bool renorm, hipStream_t stream) {
  const dim3 grid((unsigned)((T + kWavesPerBlock - 1) / kWavesPerBlock));
  const dim3 block(64 * kWavesPerBlock);
  using R = typename ScoreIn<IT>::raw;
  const R* g = reinterpret_cast<const R*>(gating);
#define MMI_ROUTER_LAUNCH(V)                                                                  \
  hipLaunchKernelGGL((topk_gating_kernel<IT, V, SF, OT>), grid, block, 0, stream, g, bias, w, \
                     ids, tei, T, E, k, (int)renorm)
  const int vpl = (E + 63) / 64;
  if (vpl <= 1) MMI_ROUTER_LAUNCH(1);
  else if (vpl <= 2) MMI_ROUTER_LAUNCH(2);
  else if (vpl <= 4) MMI_ROUTER_LAUNCH(4);
  else if (vpl <= 8) MMI_ROUTER_LAUNCH(8);
  else if (vpl <= 16) MMI_ROUTER_LAUNCH(16);
  else if (vpl <= 32) MMI_ROUTER_LAUNCH(32);
  else MMI_ROUTER_LAUNCH(64);
#undef MMI_ROUTER_LAUNCH
  return hipGetLastError();
}

template <int SF, class OT>
hipError_t launch_in(int in_kind, const void* gating, const float* bias, float* w, OT* ids,
                     int* tei, int64_t T, int E, int k, bool renorm, hipStream_t stream) {
  switch (in_kind) {
    case 0: return launch_vpl<F16, SF, OT>(gating, bias, w, ids, tei, T, E, k, renorm, stream);
    case 1: return launch_vpl<BF16, SF, OT>(gating, bias, w, ids, tei, T, E, k, renorm, stream);
    default: return launch_vpl<float, SF, OT>(gating, bias, w, ids, tei, T, E, k, renorm, stream);
  }
}

}  // namespace

hipError_t launch_topk_gating(bool sigmoid, int in_kind, const void* gating, const float* bias,
                              float* weights, void* ids, int ids_kind, int* tei, int64_t T, int E,
                              int k, bool renorm, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  if (ids_kind == 2) {
    int64_t* o = reinterpret_cast<int64_t*>(ids);
    return sigmoid ? launch_in<kSigmoid>(in_kind, gating, bias, weights, o, tei, T, E, k, renorm, stream)
                   : launch_in<kSoftmax>(in_kind, gating, bias, weights, o, tei, T, E, k, renorm, stream);
  }
  if (ids_kind == 1) {
    uint32_t* o = reinterpret_cast<uint32_t*>(ids);
    return sigmoid ? launch_in<kSigmoid>(in_kind, gating, bias, weights, o, tei, T, E, k, renorm, stream)
                   : launch_in<kSoftmax>(in_kind, gating, bias, weights, o, tei, T, E, k, renorm, stream);
  }
  int32_t* o = reinterpret_cast<int32_t*>(ids);
  return sigmoid ? launch_in<kSigmoid>(in_kind, gating, bias, weights, o, tei, T, E, k, renorm, stream)
                 : launch_in<kSoftmax>(in_kind, gating, bias, weights, o, tei, T, E, k, renorm, stream);
}

hipError_t launch_grouped_topk(int scoring, int in_kind, int bias_kind, const void* scores,
                               const void* bias, float* values, int* ids, int64_t T, int E,
                               int n_group, int topk_group, int k, bool renorm, float rsf,
                               hipStream_t stream) {
  if (T == 0) return hipSuccess;
  return scoring == kSigmoid
             ? launch_grouped_in<kSigmoid>(in_kind, bias_kind, scores, bias, values, ids, T, E,
                                           n_group, topk_group, k, renorm, rsf, stream)
             : launch_grouped_in<kScoreNone>(in_kind, bias_kind, scores, bias, values, ids, T, E,
                                           n_group, topk_group, k, renorm, rsf, stream);
}

}  // namespace mmi
