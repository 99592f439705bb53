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

// ---------------------------------------------------------------------------------------
// 8-bit-activation layout (is_a_8bit; reference gptq_marlin_repack.cu:225-335 and
// awq_marlin_repack.cu:165-270).  The weights are cut into 32 x 32 (k x n) tiles, k tiles
// outer, each tile 32 * 32 / pack words.  Within a tile, word group (thread th = 0..31,
// n8 slice s = 0..3) is the B fragment of an m16n8k32 8-bit tensor-core MMA for columns
// 16 * (s / 2) + 8 * (s % 2) + th / 4: rows k0 = 4 * (th % 4) + {0..3} and k0 + 16 + {0..3}.
//   4-bit: one word at th * 4 + s, nibble i = code(k0 + i / 2 + 16 * (i % 2));
//   8-bit: two words at th * 8 + 2 * s + h, byte i = code(k0 + 16 * h + i).
// One thread produces one output word; AWQ sources are read through the interleave slot
// of the column, as in awq_repack_kernel.
// ---------------------------------------------------------------------------------------
template <int BITS, bool AWQ>
__global__ void a8_repack_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ out,
                                 int64_t size_k, int64_t size_n, int64_t total_words) {
  constexpr int PACK = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1;
  constexpr int TILE_WORDS = 32 * 32 / PACK;
  const int64_t n_tiles = size_n / 32;
  auto code = [&](int64_t k, int64_t n) -> uint32_t {
    if constexpr (AWQ) {
      const int c = (int)(n % PACK);
      const int slot = BITS == 4 ? (c >> 1) + ((c & 1) << 2) : (c >> 1) + ((c & 1) << 1);
      return (src[k * (size_n / PACK) + n / PACK] >> (slot * BITS)) & MASK;
    } else {
      return (src[(k / PACK) * size_n + n] >> ((k % PACK) * BITS)) & MASK;
    }
  };
  for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < total_words;
       w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tile = w / TILE_WORDS;
    const int r = (int)(w - tile * TILE_WORDS);
    const int64_t kt = tile / n_tiles;
    const int64_t nt = tile - kt * n_tiles;
    const int th = BITS == 4 ? r >> 2 : r >> 3;
    const int s = BITS == 4 ? r & 3 : (r >> 1) & 3;
    const int h = BITS == 4 ? 0 : r & 1;
    const int64_t n = nt * 32 + 16 * (s >> 1) + 8 * (s & 1) + (th >> 2);
    const int64_t k0 = kt * 32 + 4 * (th & 3);
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < PACK; ++i) {
      const int64_t k = BITS == 4 ? k0 + (i >> 1) + 16 * (i & 1) : k0 + 16 * h + i;
      v |= code(k, n) << (i * BITS);
    }
    out[w] = v;
  }
}

// ---------------------------------------------------------------------------------------
// marlin_int4_fp8_preprocess (reference marlin_int4_fp8_preprocess.cu:8-56): every 4-bit
// code v becomes v - z if v >= z, else 15 - v, with z = 8 (no zero points) or the code's
// AWQ zero point (same word column, same nibble, row k / group_size).  In place is allowed.
// ---------------------------------------------------------------------------------------
__global__ void int4_fp8_preprocess_kernel(const uint32_t* q, uint32_t* out,
                                           const uint32_t* __restrict__ zeros, int64_t words,
                                           int64_t row_words, int group_size) {
  for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < words;
       w += (int64_t)gridDim.x * blockDim.x) {
    uint32_t v = q[w];
    uint32_t z = 0x88888888u;
    if (zeros != nullptr) {
      const int64_t row = w / row_words;
      z = zeros[(row / group_size) * row_words + (w - row * row_words)];
    }
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t x = (v >> (4 * i)) & 15u;
      const uint32_t zz = (z >> (4 * i)) & 15u;
      r |= (x >= zz ? x - zz : 15u - x) << (4 * i);
    }
    out[w] = r;
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

hipError_t launch_a8_repack(const uint32_t* src, bool awq, uint32_t* out, int64_t size_k,
                            int64_t size_n, int bits, hipStream_t stream) {
  const int64_t total = size_k * size_n / (32 / bits);
  const int grid = repack_grid(total);
  if (bits == 4) {
    if (awq)
      hipLaunchKernelGGL((a8_repack_kernel<4, true>), dim3(grid), dim3(256), 0, stream, src, out,
                         size_k, size_n, total);
    else
      hipLaunchKernelGGL((a8_repack_kernel<4, false>), dim3(grid), dim3(256), 0, stream, src, out,
                         size_k, size_n, total);
  } else {
    if (awq)
      hipLaunchKernelGGL((a8_repack_kernel<8, true>), dim3(grid), dim3(256), 0, stream, src, out,
                         size_k, size_n, total);
    else
      hipLaunchKernelGGL((a8_repack_kernel<8, false>), dim3(grid), dim3(256), 0, stream, src, out,
                         size_k, size_n, total);
  }
  return hipGetLastError();
}

hipError_t launch_int4_fp8_preprocess(const uint32_t* q, uint32_t* out, const uint32_t* zeros,
                                      int64_t words, int64_t row_words, int group_size,
                                      hipStream_t stream) {
  const int grid = repack_grid(words);
  hipLaunchKernelGGL(int4_fp8_preprocess_kernel, dim3(grid), dim3(256), 0, stream, q, out, zeros,
                     words, row_words, group_size);
  return hipGetLastError();
}

}  // namespace mmi
