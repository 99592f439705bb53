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
    case FMT_FP8: return launch_dequant_fmt<FMT_FP8>(p, bf16, o, gs_mode, stream);
    case FMT_MXFP4: return launch_dequant_fmt<FMT_MXFP4>(p, bf16, o, gs_mode, stream);
    case FMT_NVFP4: return launch_dequant_fmt<FMT_NVFP4>(p, bf16, o, gs_mode, stream);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------
// moe_align_block_size (reference moe_align_sum_kernels.cu:81-181, 291-320), one workgroup
// of 1024 threads.  Unlike the reference's atomic scatter, placement is deterministic:
// route indices of one expert appear in ascending order.  Rounds of 1024 indices are placed
// in index order; inside a round each wavefront ranks its lanes per expert with one ballot
// per expert-id bit and wavefronts are ordered by a per-expert prefix over per-wave counts
// kept in LDS.
// ---------------------------------------------------------------------------------------
template <typename IdT>
__global__ __launch_bounds__(1024) void moe_align_kernel(
    const IdT* __restrict__ topk, int64_t numel, int E, int bs, int* __restrict__ sorted,
    int64_t sorted_numel, int* __restrict__ expert_ids, int64_t expert_ids_numel,
    int* __restrict__ post_pad, const int* __restrict__ expert_map, int has_map) {
  extern __shared__ int smem[];
  int* counts = smem;             // [E]
  int* cursor = counts + E;       // [E + 1] exclusive padded prefix, then running cursor
  uint8_t* wave_cnt = reinterpret_cast<uint8_t*>(cursor + E + 1);  // [16][E]
  __shared__ int scan_tmp[1024];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ebits = E > 1 ? 32 - __clz(E - 1) : 1;  // bits of the largest expert id

  auto mapped = [&](int64_t i) -> int {
    int64_t e = (int64_t)topk[i];
    if (e < 0 || e >= E) return -1;
    int me = (int)e;
    if (has_map) {
      me = expert_map[me];
      if (me < 0 || me >= E) return -1;
    }
    return me;
  };

  for (int e = tid; e < E; e += 1024) counts[e] = 0;
  __syncthreads();
  for (int64_t i = tid; i < numel; i += 1024) {
    const int e = mapped(i);
    if (e >= 0) atomicAdd(&counts[e], 1);
  }
  __syncthreads();

  // exclusive scan of padded counts (E <= 1024: one value per thread)
  int v = 0;
  if (tid < E) v = (counts[tid] + bs - 1) / bs * bs;
  scan_tmp[tid] = v;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int add = tid >= off ? scan_tmp[tid - off] : 0;
    __syncthreads();
    scan_tmp[tid] += add;
    __syncthreads();
  }
  const int incl = scan_tmp[tid];
  if (tid < E) cursor[tid] = incl - v;
  if (tid == E - 1) cursor[E] = incl;
  __syncthreads();
  const int total = cursor[E];
  if (tid == 0) post_pad[0] = total;

  // expert_ids
  for (int e = tid; e < E; e += 1024) {
    for (int b = cursor[e] / bs; b < cursor[e + 1] / bs; ++b)
      if (b < expert_ids_numel) expert_ids[b] = e;
  }
  for (int64_t b = total / bs + tid; b < expert_ids_numel; b += 1024) expert_ids[b] = -1;

  // sentinel fill, then placement
  for (int64_t i = tid; i < sorted_numel; i += 1024) sorted[i] = (int)numel;
  __syncthreads();

  for (int64_t base = 0; base < numel; base += 1024) {
    const int64_t i = base + tid;
    const int e = i < numel ? mapped(i) : -1;
    for (int x = lane; x < E; x += 64) wave_cnt[wave * E + x] = 0;
    // lanes holding the same expert: intersect, over the id's bits, the ballots that agree
    // with this lane's bit (no per-expert loop)
    uint64_t same = __ballot(e >= 0);
    for (int bit = 0; bit < ebits; ++bit) {
      const int set = (e >> bit) & 1;
      const uint64_t m = __ballot(set);
      same &= set ? m : ~m;
    }
    const uint64_t before = same & ((1ull << lane) - 1);
    const int rank = __popcll(before);
    if (e >= 0 && before == 0) wave_cnt[wave * E + e] = (uint8_t)__popcll(same);
    __syncthreads();
    if (e >= 0) {
      int pos = cursor[e] + rank;
      for (int w = 0; w < wave; ++w) pos += wave_cnt[w * E + e];
      if (pos < sorted_numel) sorted[pos] = (int)i;
    }
    __syncthreads();
    for (int x = tid; x < E; x += 1024) {
      int add = 0;
      for (int w = 0; w < 16; ++w) add += wave_cnt[w * E + x];
      cursor[x] += add;
    }
    __syncthreads();
  }
}

hipError_t launch_moe_align(const void* topk, bool is64, int64_t numel, int E, int bs, int* sorted,
                            int64_t sorted_numel, int* expert_ids, int64_t expert_ids_numel,
                            int* post_pad, const int* expert_map, hipStream_t stream) {
  const size_t smem = (size_t)(2 * E + 1) * sizeof(int) + (size_t)16 * E;
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
// moe_sum: out[t, h] = sum_k in[t, k, h], fp32 accumulation, one rounding.
// ---------------------------------------------------------------------------------------
template <class AT>
__global__ void moe_sum_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                               int64_t tokens, int topk, int64_t hidden) {
  const int64_t t = blockIdx.y;
  for (int64_t h = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; h < hidden;
       h += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int k = 0; k < topk; ++k) s += raw16_to_float(in[(t * topk + k) * hidden + h], AT{});
    out[t * hidden + h] = to_raw16(s, AT{});
  }
}

hipError_t launch_moe_sum(const void* in, bool bf16, int64_t tokens, int topk, int64_t hidden,
                          void* out, hipStream_t stream) {
  if (tokens == 0 || hidden == 0) return hipSuccess;
  unsigned gx = (unsigned)((hidden + 255) / 256);
  if (gx > 64) gx = 64;
  dim3 grid(gx, (unsigned)tokens);
  const uint16_t* i16 = reinterpret_cast<const uint16_t*>(in);
  uint16_t* o16 = reinterpret_cast<uint16_t*>(out);
  if (bf16)
    hipLaunchKernelGGL((moe_sum_kernel<BF16>), grid, dim3(256), 0, stream, i16, o16, tokens, topk,
                       hidden);
  else
    hipLaunchKernelGGL((moe_sum_kernel<F16>), grid, dim3(256), 0, stream, i16, o16, tokens, topk,
                       hidden);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// silu_and_mul: out[r, j] = silu(x[r, j]) * x[r, d + j], rounded as the reference's torch
// expression F.silu(gate) * up rounds: silu to the element type, then the product.
// ---------------------------------------------------------------------------------------
template <class AT>
__device__ __forceinline__ float silu_mul1(uint32_t g_raw, uint32_t u_raw) {
  const float g = raw16_to_float(g_raw & 0xffffu, AT{});
  const float u = raw16_to_float(u_raw & 0xffffu, AT{});
  const float s = raw16_to_float(to_raw16(g / (1.0f + expf(-g)), AT{}), AT{});
  return s * u;
}

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
