// repack.hip -- GPTQ / AWQ packed weights -> tile-chunk layout (device_common.h).
//
// One thread produces one output word.  GPTQ words already hold consecutive k of one column
// in natural order (tests/helpers.py:401-426), so without act-order the repack is a pure
// word gather.  AWQ words hold consecutive columns of one k in AWQ interleave order
// (tests/helpers.py:548-562), so each output word gathers one value from pack source words.
// Act-order (perm) gathers every value from row perm[k] of the GPTQ source
// (reference gptq_marlin_repack.cu:8-121, has_perm path).
#include "device_common.h"
#include "host_common.h"

namespace mmi {

// Decode an output word index into (n, k of its first value); inverse of
// layout_word_index().
__device__ __forceinline__ void decode_word(int bits, int64_t size_k, int64_t size_n, int64_t w,
                                            int64_t& n, int64_t& k) {
  const int64_t tiles = size_n >> 4;
  const int64_t kc = chunk_k(bits);
  const int64_t full = size_k / kc;
  const int64_t full_words = full * tiles * 256;
  int64_t t, c, lane, j;
  if (w < full_words) {
    const int64_t chunk = w >> 8;
    c = chunk / tiles;
    t = chunk - c * tiles;
    lane = (w >> 2) & 63;
    j = w & 3;
  } else {
    const int64_t wpl = (size_k - full * kc) / 32 * (bits / 4);
    const int64_t r = w - full_words;
    const int64_t tl = r / wpl;  // t * 64 + lane
    j = r - tl * wpl;
    t = tl >> 6;
    lane = tl & 63;
    c = full;
  }
  const int64_t g = lane >> 4;
  n = t * 16 + (lane & 15);
  if (bits == 4) {
    k = c * kc + 32 * j + 8 * g;
  } else {
    k = c * kc + 32 * (j >> 1) + 8 * g + 4 * (j & 1);
  }
}

template <int BITS, bool HAS_PERM>
__global__ void gptq_repack_kernel(const uint32_t* __restrict__ src, const int* __restrict__ perm,
                                   uint32_t* __restrict__ out, int64_t size_k, int64_t size_n,
                                   int64_t total_words) {
  constexpr int PACK = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1;
  for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < total_words;
       w += (int64_t)gridDim.x * blockDim.x) {
    int64_t n, k;
    decode_word(BITS, size_k, size_n, w, n, k);
    uint32_t v;
    if constexpr (!HAS_PERM) {
      v = src[(k / PACK) * size_n + n];
    } else {
      v = 0;
#pragma unroll
      for (int i = 0; i < PACK; ++i) {
        const int64_t sk = perm[k + i];
        const uint32_t sw = src[(sk / PACK) * size_n + n];
        v |= ((sw >> ((sk % PACK) * BITS)) & MASK) << (i * BITS);
      }
    }
    out[w] = v;
  }
}

template <int BITS>
__global__ void awq_repack_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ out,
                                  int64_t size_k, int64_t size_n, int64_t total_words) {
  constexpr int PACK = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1;
  // AWQ slot s of a word holds column 8*np + {0,2,4,6,1,3,5,7}[s] (4-bit) or
  // 4*np + {0,2,1,3}[s] (8-bit); these tables give the slot of column offset c.
  for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < total_words;
       w += (int64_t)gridDim.x * blockDim.x) {
    int64_t n, k;
    decode_word(BITS, size_k, size_n, w, n, k);
    const int c = (int)(n % PACK);
    int slot;
    if constexpr (BITS == 4) {
      slot = (c >> 1) + ((c & 1) << 2);  // inverse of {0,2,4,6,1,3,5,7}
    } else {
      slot = (c >> 1) + ((c & 1) << 1);  // inverse of {0,2,1,3}
    }
    const int64_t np = n / PACK;
    const int64_t row_words = size_n / PACK;
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < PACK; ++i) {
      const uint32_t sw = src[(k + i) * row_words + np];
      v |= ((sw >> (slot * BITS)) & MASK) << (i * BITS);
    }
    out[w] = v;
  }
}

static int repack_grid(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

hipError_t launch_gptq_repack(const uint32_t* src, const int* perm, uint32_t* out, int64_t size_k,
                              int64_t size_n, int bits, hipStream_t stream) {
  const int64_t total = size_k * size_n / (32 / bits);
  const int grid = repack_grid(total);
  if (bits == 4) {
    if (perm)
      hipLaunchKernelGGL((gptq_repack_kernel<4, true>), dim3(grid), dim3(256), 0, stream, src, perm,
                         out, size_k, size_n, total);
    else
      hipLaunchKernelGGL((gptq_repack_kernel<4, false>), dim3(grid), dim3(256), 0, stream, src,
                         perm, out, size_k, size_n, total);
  } else {
    if (perm)
      hipLaunchKernelGGL((gptq_repack_kernel<8, true>), dim3(grid), dim3(256), 0, stream, src, perm,
                         out, size_k, size_n, total);
    else
      hipLaunchKernelGGL((gptq_repack_kernel<8, false>), dim3(grid), dim3(256), 0, stream, src,
                         perm, out, size_k, size_n, total);
  }
  return hipGetLastError();
}

hipError_t launch_awq_repack(const uint32_t* src, uint32_t* out, int64_t size_k, int64_t size_n,
                             int bits, hipStream_t stream) {
  const int64_t total = size_k * size_n / (32 / bits);
  const int grid = repack_grid(total);
  if (bits == 4)
    hipLaunchKernelGGL((awq_repack_kernel<4>), dim3(grid), dim3(256), 0, stream, src, out, size_k,
                       size_n, total);
  else
    hipLaunchKernelGGL((awq_repack_kernel<8>), dim3(grid), dim3(256), 0, stream, src, out, size_k,
                       size_n, total);
  return hipGetLastError();
}

}  // namespace mmi
