// device_common.h -- types, weight layout, dequant routines and MFMA wrappers for gfx950.
//
// Weight layout ("chunk-major layout"), shared by the repack, dequant and GEMM kernels.
// The packed weight buffer keeps the reference's container shape [K/16, N*16/pack] int32
// (vllm/_custom_ops.py:1187-1193) but orders words for 64-wide wavefronts feeding
// v_mfma_f32_16x16x32_{f16,bf16}:
//   * Columns are split into T = N/16 n16 tiles and K into chunks of KC = 128 k (4-bit) or
//     KC = 64 k (8-bit).  One (tile, chunk) is 1 KiB = 64 lanes x 4 words.  Lane l owns
//     column 16t + l%16 and lane-group g = l/16; its 4 words are consecutive, so one
//     dwordx4 per lane loads the whole chunk with a fully coalesced 1 KiB wave access.
//   * Chunks are stored chunk-major: chunk c of tile t sits at word (c*T + t) * 256.  At
//     any K step every tile's chunk is adjacent, so all waves of the chip read one
//     contiguous region instead of thousands of strided streams.
//   * Word j of lane l holds, for 4-bit: the 8 values k = c*128 + 32*j + 8*g + [0..7]
//     (k32 block j of the chunk); for 8-bit: the 4 values
//     k = c*64 + 32*(j/2) + 8*g + 4*(j%2) + [0..3].  Values sit in natural order, value i in
//     bits [i*bits, (i+1)*bits).
//   * That is exactly the B operand of one 16x16x32 MFMA: lane l supplies column l%16 and
//     k-slice 8*g..8*g+7 of a 32-deep block.  The A operand uses the same k-slice per lane.
//   * K % KC != 0 leaves a tail of (K % KC)/32 k32 blocks per tile, stored after all full
//     chunks, tile-major, J tail words per lane, lane-major.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmi {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

// Activation / output element tags.
struct F16 {
  static constexpr int kId = 0;
};
struct BF16 {
  static constexpr int kId = 1;
};

// Weight formats handled by the kernels.
enum Fmt : int {
  FMT_U4B8 = 0,   // uint4, bias 8 (GPTQ symmetric)
  FMT_U4 = 1,     // uint4 + float zero point (AWQ)
  FMT_U8B128 = 2, // uint8, bias 128
  FMT_U8 = 3,     // uint8 + float zero point
  FMT_FP8 = 4,    // float8_e4m3fn, scales carry the x256 exponent fold
  FMT_MXFP4 = 5,  // float4_e2m1f + float8_e8m0fnu scale per 32
  FMT_NVFP4 = 6,  // float4_e2m1f + S0E5M3 scale per 16 + fp32 global scale
  FMT_U4Z = 7,    // uint4 + integer zero point (16-bit codes expanded by the launcher)
  FMT_U8Z = 8,    // uint8 + integer zero point
};

__host__ __device__ constexpr int fmt_bits(int f) {
  return (f == FMT_U8B128 || f == FMT_U8 || f == FMT_U8Z || f == FMT_FP8) ? 8 : 4;
}
__host__ __device__ constexpr bool fmt_int_zero(int f) { return f == FMT_U4Z || f == FMT_U8Z; }
__host__ __device__ constexpr bool fmt_has_zp(int f) {
  return f == FMT_U4 || f == FMT_U8 || fmt_int_zero(f);
}
__host__ __device__ constexpr bool fmt_byte_scale(int f) {
  return f == FMT_MXFP4 || f == FMT_NVFP4;
}

// ---------------------------------------------------------------------------------------
// Layout index math (host and device).
// ---------------------------------------------------------------------------------------
__host__ __device__ inline int64_t tile_words(int bits, int64_t size_k) {
  return size_k * 16 / (32 / bits);
}
__host__ __device__ inline int chunk_k(int bits) { return bits == 4 ? 128 : 64; }

// Word index of the word holding values (n, k..k+pack-1), k a multiple of pack.
__host__ __device__ inline int64_t layout_word_index(int bits, int64_t size_k, int64_t size_n,
                                                     int64_t n, int64_t k) {
  const int64_t tiles = size_n >> 4;
  const int64_t t = n >> 4;
  const int64_t nl = n & 15;
  const int64_t kc = chunk_k(bits);
  const int64_t full = size_k / kc;
  const int64_t c = k / kc;
  const int64_t kin = k - c * kc;  // k inside chunk
  const int64_t blk = kin >> 5;    // k32 block inside chunk
  const int64_t g = (kin >> 3) & 3;
  const int64_t lane = g * 16 + nl;
  const int64_t j = (bits == 4) ? blk : blk * 2 + ((kin >> 2) & 1);
  if (c < full) return (c * tiles + t) * 256 + lane * 4 + j;
  const int64_t wpl = (size_k - full * kc) / 32 * (bits / 4);  // tail words per lane
  return full * tiles * 256 + (t * 64 + lane) * wpl + j;
}

// ---------------------------------------------------------------------------------------
// Scalar conversions.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float raw16_to_float(uint32_t raw, F16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)raw);
}
__device__ __forceinline__ float raw16_to_float(uint32_t raw, BF16) {
  return __builtin_bit_cast(float, raw << 16);
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi, F16) {
  f16x2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi, BF16) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t to_raw16(float v, F16) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}
__device__ __forceinline__ uint16_t to_raw16(float v, BF16) {
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}

// e8m0 byte -> 2^(e-127) as fp32 (e = 255 -> NaN).
__device__ __forceinline__ float e8m0_to_float(uint32_t e) {
  uint32_t bits = e == 0 ? 0x00400000u : (e == 255 ? 0x7fc00000u : (e << 23));
  return __builtin_bit_cast(float, bits);
}
// S0E5M3 byte b (the reference's NVFP4 scale re-encoding, marlin_utils_fp4.py:83-110):
// fp16 bits (b << 7) hold scale*2^7*sf.  Returns scale*sf = fp16(b<<7) * 2^-7 as fp32.
__device__ __forceinline__ float s0e5m3_to_float_div128(uint32_t b) {
  return b == 0 ? 0.0f : __builtin_bit_cast(float, (b << 20) + (105u << 23));
}

// ---------------------------------------------------------------------------------------
// Per-group dequant constants ("meta") and operand dequantization.
//
// Integer formats use the fp16 magic-number trick: (nibble | 0x6400) is the fp16 value
// 1024 + q (or 1024 + 16q for the odd nibble of a byte).  v_fma_mix_f32 widens that half
// exactly and computes x*s' + c in one fused step; c is chosen so the result is exactly
// q*s - zp (or (q - bias)*s).  Every such value has at most 22 significant bits, so the
// fp32 result is exact and the single conversion to the activation dtype is the only
// rounding -- the reference semantics rnd(q*s - zp) / rnd((q - bias)*s)
// (tests/helpers.py:1094-1133, 1576-1641; dequant.h:131-328).
// ---------------------------------------------------------------------------------------
struct Meta {
  float s;    // scale for values at 1024 + q
  float s16;  // scale/16 for values at 1024 + 16q
  float c1;   // offset for 1024 + q
  float c16;  // offset for 1024 + 16q
};

// Raw metadata for one (group, column) as loaded: the scale bits (16-bit, or the fp4 scale
// byte) and the float zero point bits.  The two halves stay in separate registers until
// use, so a prefetch of the next step never has to wait for them.
struct MetaRaw {
  uint32_t s;
  uint32_t z;
};

// Zero point z*s as fp32 for uint4/uint8: the float zero point as stored, or (integer-zero
// formats) the code times the scale (exact: <= 8 + 11 significant bits), so that the dequant
// below yields the single rounding of the exact (q - z) * s.
template <int FMT, class AT>
__device__ __forceinline__ float zero_point_value(uint32_t z, float s) {
  if constexpr (fmt_int_zero(FMT)) return (float)(z & 0xffu) * s;
  else return raw16_to_float(z & 0xffff, AT{});
}

// A scale byte loaded into a prefetch ring, made opaque at the point of use.  The fp4 scale
// decodings compare the byte with constants; left visible, the scheduler moves those compares
// up to the byte's load (their i1 results live in SGPRs, which frees the byte's VGPR), and
// the wave then waits for a load it has just issued instead of one from two steps before
// (cfg4 shape, MXFP4 M = 1 / 64: 8.3 / 25.2 -> 7.9 / 23.0 us).
__device__ __forceinline__ MetaRaw use_raw(MetaRaw raw) {
  asm volatile("" : "+v"(raw.s));
  return raw;
}

template <int FMT, class AT>
__device__ __forceinline__ Meta make_meta(MetaRaw raw) {
  Meta m;
  if constexpr (FMT == FMT_MXFP4 || FMT == FMT_NVFP4) raw = use_raw(raw);
  if constexpr (FMT == FMT_MXFP4) {
    m.s = e8m0_to_float(raw.s & 0xff);
    m.s16 = m.c1 = m.c16 = 0.f;
  } else if constexpr (FMT == FMT_NVFP4) {
    // v_cvt_scalef32_pk_*_fp4 applies only the exponent of its scale operand, so the scale
    // s*sf = 2^E * (1 + m/8) is split: s = 2^E goes to the conversion, s16 carries the full
    // value (bf16 path) and c1 holds (1 + m/8) as an f16 pair (f16 path).
    const float full = s0e5m3_to_float_div128(raw.s & 0xff);
    const uint32_t fb = __builtin_bit_cast(uint32_t, full);
    m.s = __builtin_bit_cast(float, fb & 0xff800000u);
    m.s16 = full;
    const _Float16 mant = (_Float16)__builtin_bit_cast(float, (fb & 0x007fffffu) | 0x3f800000u);
    const f16x2_t mm = {mant, mant};
    m.c1 = __builtin_bit_cast(float, mm);
    m.c16 = 0.f;
  } else if constexpr (FMT == FMT_FP8) {
    // Dequant is fp8 * (s / 256) (tests/helpers.py:1117-1121).  bf16 path: s/256 in fp32;
    // fp16 path: the stored fp16 scale s as a packed pair in c1.
    m.s = raw16_to_float(raw.s & 0xffff, AT{}) * 0.00390625f;
    m.s16 = 0.f;
    m.c1 = __builtin_bit_cast(float, (raw.s & 0xffffu) | (raw.s << 16));
    m.c16 = 0.f;
  } else {
    const float s = raw16_to_float(raw.s & 0xffff, AT{});
    m.s = s;
    m.s16 = s * 0.0625f;
    if constexpr (FMT == FMT_U4B8) {
      m.c1 = -1032.0f * s;  // (1024 + q)*s - 1032 s = (q - 8) s
      m.c16 = -72.0f * s;   // (1024 + 16q)*s/16 - 72 s = (q - 8) s
    } else if constexpr (FMT == FMT_U8B128) {
      m.c1 = -1152.0f * s;  // (1024 + q)*s - 1152 s = (q - 128) s
      m.c16 = 0.f;
    } else {
      const float z = zero_point_value<FMT, AT>(raw.z, s);
      m.c1 = __builtin_fmaf(-1024.0f, s, -z);  // exact: |1024 s + z| has <= 22 bits
      m.c16 = __builtin_fmaf(-64.0f, s, -z);
    }
  }
  return m;
}

// (x & MASK) | bits in one v_and_or_b32.  A VOP3 instruction on gfx9 reads no literal and
// at most one SGPR, so the mask has to sit in a VGPR the optimizer cannot fold back into a
// literal (which would split the op into v_and + v_or): MASK | vz, where vz is a VGPR
// holding zero that the compiler cannot prove is zero (opaque_zero()).  The instruction is
// compiler-generated on purpose: results that feed MFMA operands need the wait states the
// hazard recognizer inserts after a VALU write, which it never does for inline assembly.
template <uint32_t MASK>
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t bits, uint32_t vz) {
  return (x & (MASK | vz)) | bits;
}
// Same, for a result consumed half by half (v_fma_mix_f32 op_sel): an empty asm with a
// read-write VGPR operand emits nothing but hides the value from the optimizer, which would
// otherwise narrow the op per half and split it back into v_and + v_or.  Only for values
// that do not feed an MFMA directly.
template <uint32_t MASK>
__device__ __forceinline__ uint32_t and_or_halves(uint32_t x, uint32_t bits, uint32_t vz) {
  uint32_t r = and_or<MASK>(x, bits, vz);
  asm("" : "+v"(r));
  return r;
}
// Zero in a VGPR, from a kernel argument that is always zero.
__device__ __forceinline__ uint32_t opaque_zero(int zero_arg) {
  return threadIdx.x & (uint32_t)zero_arg;
}

__device__ __forceinline__ float h_lo(uint32_t x) {
  return (float)__builtin_bit_cast(f16x2_t, x)[0];
}
__device__ __forceinline__ float h_hi(uint32_t x) {
  return (float)__builtin_bit_cast(f16x2_t, x)[1];
}

// Dequantize the MFMA B operand of one lane: 8 consecutive k of one column.
// 4-bit formats read w0 only, 8-bit formats read w0 (k0..3) and w1 (k4..7).
template <int FMT, class AT>
__device__ __forceinline__ u32x4_t dequant_operand(uint32_t w0, uint32_t w1, const Meta& m,
                                                 uint32_t vz) {
  u32x4_t r;
  if constexpr (FMT == FMT_U4B8 || FMT == FMT_U4 || FMT == FMT_U4Z) {
    const uint32_t x0 = and_or_halves<0x000f000fu>(w0, 0x64006400u, vz);  // k0, k4  : 1024 + q
    const uint32_t x1 = and_or_halves<0x00f000f0u>(w0, 0x64006400u, vz);  // k1, k5  : 1024 + 16q
    const uint32_t t = w0 >> 8;
    const uint32_t x2 = and_or_halves<0x000f000fu>(t, 0x64006400u, vz);  // k2, k6
    const uint32_t x3 = and_or_halves<0x00f000f0u>(t, 0x64006400u, vz);  // k3, k7
    const float e0 = __builtin_fmaf(h_lo(x0), m.s, m.c1);
    const float e4 = __builtin_fmaf(h_hi(x0), m.s, m.c1);
    const float e1 = __builtin_fmaf(h_lo(x1), m.s16, m.c16);
    const float e5 = __builtin_fmaf(h_hi(x1), m.s16, m.c16);
    const float e2 = __builtin_fmaf(h_lo(x2), m.s, m.c1);
    const float e6 = __builtin_fmaf(h_hi(x2), m.s, m.c1);
    const float e3 = __builtin_fmaf(h_lo(x3), m.s16, m.c16);
    const float e7 = __builtin_fmaf(h_hi(x3), m.s16, m.c16);
    r[0] = pack2(e0, e1, AT{});
    r[1] = pack2(e2, e3, AT{});
    r[2] = pack2(e4, e5, AT{});
    r[3] = pack2(e6, e7, AT{});
  } else if constexpr (FMT == FMT_U8B128 || FMT == FMT_U8 || FMT == FMT_U8Z) {
    const uint32_t a0 = and_or_halves<0x00ff00ffu>(w0, 0x64006400u, vz);       // k0, k2
    const uint32_t a1 = and_or_halves<0x00ff00ffu>(w0 >> 8, 0x64006400u, vz);  // k1, k3
    const uint32_t b0 = and_or_halves<0x00ff00ffu>(w1, 0x64006400u, vz);       // k4, k6
    const uint32_t b1 = and_or_halves<0x00ff00ffu>(w1 >> 8, 0x64006400u, vz);  // k5, k7
    r[0] = pack2(__builtin_fmaf(h_lo(a0), m.s, m.c1), __builtin_fmaf(h_lo(a1), m.s, m.c1),
                 AT{});
    r[1] = pack2(__builtin_fmaf(h_hi(a0), m.s, m.c1), __builtin_fmaf(h_hi(a1), m.s, m.c1),
                 AT{});
    r[2] = pack2(__builtin_fmaf(h_lo(b0), m.s, m.c1), __builtin_fmaf(h_lo(b1), m.s, m.c1),
                 AT{});
    r[3] = pack2(__builtin_fmaf(h_hi(b0), m.s, m.c1), __builtin_fmaf(h_hi(b1), m.s, m.c1),
                 AT{});
  } else if constexpr (FMT == FMT_FP8 && AT::kId == 0) {
    // fp16: e4m3fn * 2^-8 -> fp16 exactly (hardware scaled conversion, power-of-two scale),
    // then one packed fp16 multiply by s: a single rounding of the exact fp8 * s / 256.
    const f16x2_t s2 = __builtin_bit_cast(f16x2_t, m.c1);
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 0.00390625f, false) * s2);
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 0.00390625f, true) * s2);
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 0.00390625f, false) * s2);
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 0.00390625f, true) * s2);
  } else if constexpr (FMT == FMT_FP8) {
    // bf16: OCP e4m3fn -> fp32 exactly, times s/256 (exact: <= 15 significant bits), one
    // rounding in the conversion to bf16.
    const f32x2_t p0 = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false);
    const f32x2_t p1 = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
    const f32x2_t p2 = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false);
    const f32x2_t p3 = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
    r[0] = pack2(p0[0] * m.s, p0[1] * m.s, AT{});
    r[1] = pack2(p1[0] * m.s, p1[1] * m.s, AT{});
    r[2] = pack2(p2[0] * m.s, p2[1] * m.s, AT{});
    r[3] = pack2(p3[0] * m.s, p3[1] * m.s, AT{});
  } else if constexpr (FMT == FMT_NVFP4) {
    // e2m1 (<= 2 significant bits) times the e4m3-derived scale (<= 4 significant bits) is
    // exact in fp16/bf16.  fp16: convert with the power-of-two part, then one packed
    // multiply by (1 + m/8).  bf16: convert to fp32 and multiply by the full scale.
    if constexpr (AT::kId == 1) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        f32x2_t v;
        switch (b) {
          case 0: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w0, 1.0f, 0); break;
          case 1: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w0, 1.0f, 1); break;
          case 2: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w0, 1.0f, 2); break;
          default: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w0, 1.0f, 3); break;
        }
        r[b] = pack2(v[0] * m.s16, v[1] * m.s16, AT{});
      }
    } else {
      const f16x2_t mm = __builtin_bit_cast(f16x2_t, m.c1);
      r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 0) * mm);
      r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 1) * mm);
      r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 2) * mm);
      r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 3) * mm);
    }
  } else {
    // MXFP4: e2m1 pairs -> 16-bit with the hardware scaled conversion; the e8m0 scale is a
    // power of two, which is what the conversion applies (it uses only the scale's
    // exponent), so the result is exact.
    if constexpr (AT::kId == 1) {
      r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, m.s, 0));
      r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, m.s, 1));
      r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, m.s, 2));
      r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w0, m.s, 3));
    } else {
      r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 0));
      r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 1));
      r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 2));
      r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w0, m.s, 3));
    }
  }
  return r;
}

// ---------------------------------------------------------------------------------------
// Integer-operand path: scale after the MFMA.
//
// For the integer and fp8 formats the MFMA B operand can carry the code itself instead of
// the dequantized weight, and the column's scale / zero point is applied once to the fp32
// partial sum of a whole group:
//     sum_k a_k w_k = S * D - C * R,   D = sum_k a_k B_k,   R = sum_k a_k (row sum),
//   u4     B = MAGIC + q       (one v_and_or_b32 per pair: fp16 1024 + q, bf16 128 + q)
//   u8     B = 1024 + q (fp16, v_perm_b32 with the exponent byte) or q (bf16, exact)
//   fp8    B = the e4m3 value (hardware conversion, exact in fp16 and bf16)
// with (S, C) = (s, s*(MAGIC + bias)) for biased codes, (s, s*MAGIC + z) for float zero
// points and (s/256, 0) for fp8.  Every product a_k*B_k is exact in fp32, so the result
// differs from dequantize-then-multiply only by the per-weight rounding the latter applies;
// the dequantize op itself keeps the bit-exact dequant_operand() above.
// ---------------------------------------------------------------------------------------
template <int FMT, class AT>
struct IntOperand {
  static constexpr bool kEnabled = FMT == FMT_U4B8 || FMT == FMT_U4 || FMT == FMT_U8B128 ||
                                   FMT == FMT_U8 || FMT == FMT_FP8 || fmt_int_zero(FMT);
  // fp16 with a fixed code offset (uint4b8, uint8b128): one v_pk_add_f16 per register turns
  // 1024+q into the signed value q-bias exactly, so the group sums need no row-sum term
  static constexpr bool kDirect = AT::kId == 0 && (FMT == FMT_U4B8 || FMT == FMT_U8B128);
  static constexpr bool kNeedRowSum = FMT != FMT_FP8 && !kDirect;
  // code offset carried by B: the magic number of the 16-bit pattern
  static constexpr float kMagic =
      (fmt_bits(FMT) == 4 || AT::kId == 0) ? (AT::kId == 0 ? 1024.0f : 128.0f) : 0.0f;
  static constexpr uint32_t kMagicBits = AT::kId == 0 ? 0x64006400u : 0x43004300u;
  // 1.0 in both halves: B operand of the row-sum MFMA
  static constexpr uint32_t kOnes = AT::kId == 0 ? 0x3c003c00u : 0x3f803f80u;
};

struct IMeta {
  float S;  // multiplies D
  float C;  // multiplies the row sum R
};

template <int FMT, class AT>
__device__ __forceinline__ IMeta make_imeta(MetaRaw raw) {
  using IO = IntOperand<FMT, AT>;
  const float s = raw16_to_float(raw.s & 0xffff, AT{});
  if constexpr (FMT == FMT_FP8) {
    return IMeta{s * 0.00390625f, 0.0f};
  } else if constexpr (IO::kDirect) {
    return IMeta{s, 0.0f};
  } else if constexpr (FMT == FMT_U4B8) {
    return IMeta{s, s * (IO::kMagic + 8.0f)};
  } else if constexpr (FMT == FMT_U8B128) {
    return IMeta{s, s * (IO::kMagic + 128.0f)};
  } else {
    const float z = zero_point_value<FMT, AT>(raw.z, s);
    return IMeta{s, __builtin_fmaf(s, IO::kMagic, z)};
  }
}

// The 4-bit integer operand holds its 8 values in k order [0,4,1,5,2,6,3,7] (one
// v_and_or_b32 per pair, no repacking of the nibbles); the A operand is permuted to match.
__device__ __forceinline__ u32x4_t a_perm_u4(const u32x4_t& n) {
  u32x4_t r;
  r[0] = __builtin_amdgcn_perm(n[2], n[0], 0x05040100u);  // a0, a4
  r[1] = __builtin_amdgcn_perm(n[2], n[0], 0x07060302u);  // a1, a5
  r[2] = __builtin_amdgcn_perm(n[3], n[1], 0x05040100u);  // a2, a6
  r[3] = __builtin_amdgcn_perm(n[3], n[1], 0x07060302u);  // a3, a7
  return r;
}

template <int FMT, class AT>
__device__ __forceinline__ u32x4_t int_operand(uint32_t w0, uint32_t w1, uint32_t vz) {
  using IO = IntOperand<FMT, AT>;
  u32x4_t r;
  if constexpr (fmt_bits(FMT) == 4) {
    r[0] = and_or<0x000f000fu>(w0, IO::kMagicBits, vz);
    r[1] = and_or<0x000f000fu>(w0 >> 4, IO::kMagicBits, vz);
    r[2] = and_or<0x000f000fu>(w0 >> 8, IO::kMagicBits, vz);
    r[3] = and_or<0x000f000fu>(w0 >> 12, IO::kMagicBits, vz);
  } else if constexpr (FMT == FMT_FP8) {
    if constexpr (AT::kId == 0) {
      r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false));
      r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true));
      r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false));
      r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true));
    } else {
      r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false));
      r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true));
      r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false));
      r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true));
    }
  } else if constexpr (AT::kId == 0) {
    // u8, fp16: bytes [q_i, 0x64] are the fp16 value 1024 + q_i
    r[0] = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
    r[1] = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
    r[2] = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
    r[3] = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
  } else {
    // u8, bf16: q < 256 is exact in bf16
    r[0] = pack2((float)(w0 & 0xffu), (float)((w0 >> 8) & 0xffu), AT{});
    r[1] = pack2((float)((w0 >> 16) & 0xffu), (float)(w0 >> 24), AT{});
    r[2] = pack2((float)(w1 & 0xffu), (float)((w1 >> 8) & 0xffu), AT{});
    r[3] = pack2((float)((w1 >> 16) & 0xffu), (float)(w1 >> 24), AT{});
  }
  if constexpr (IO::kDirect) {
    constexpr _Float16 off = (_Float16)(-(IO::kMagic + (FMT == FMT_U4B8 ? 8.0f : 128.0f)));
    // (each element goes through a scalar: __builtin_bit_cast of a vector element
    // expression reads from the start of the vector)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t x = r[i];
      r[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, x) + f16x2_t{off, off});
    }
  }
  return r;
}

// D += A(32x16) * B(16x32) (v_mfma_f32_32x32x16: twice the work of the 16x16x32 form in
// about the same issue time on gfx950).  Lane l supplies A row l%32 / B column l%32,
// k-slice 8*(l/32).  Result lane l holds D[8*(v/4) + 4*(l/32) + v%4][l%32], v = 0..15.
__device__ __forceinline__ f32x16_t mfma32(const u32x4_t& a, const u32x4_t& b, f32x16_t c, F16) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(const u32x4_t& a, const u32x4_t& b, f32x16_t c, BF16) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Re-deals one word of two n16 tiles (x: tile t, y: tile t+1; 16-lane row g of a tile holds
// k-slice g of a 32-deep block) into the B operands of two 32x32x16 MFMAs over the 32
// columns: d0 = k-slices 0,1 (rows [x0, y0, x1, y1]), d1 = k-slices 2,3 ([x2, y2, x3, y3]).
// v_permlane16_swap gives [x0, y0, x2, y2] / [x1, y1, x3, y3]; v_permlane32_swap of those
// gives d0 / d1.
__device__ __forceinline__ void deal32(uint32_t x, uint32_t y, uint32_t& d0, uint32_t& d1) {
  const auto s16 = __builtin_amdgcn_permlane16_swap(x, y, false, false);
  const auto s32 = __builtin_amdgcn_permlane32_swap(s16[0], s16[1], false, false);
  d0 = s32[0];
  d1 = s32[1];
}

// D += A(16x32) * B(32x16).  Lane l supplies A row l%16 / B column l%16, k-slice 8*(l/16).
// Result lane l holds D[4*(l/16) + i][l%16], i = 0..3.
__device__ __forceinline__ f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, f32x4_t c, F16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, f32x4_t c,
                                          BF16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// silu(g) * u on 16-bit inputs, rounded as the reference's torch expression
// F.silu(gate) * up rounds (activation.py:45-52): silu to the element type, then the product
// (the caller rounds it).  Shared by silu_and_mul and the gated MoE epilogue, so the fused
// and the two-pass paths give the same bits.
template <class AT>
__device__ __forceinline__ float silu_mul1(uint32_t g_raw, uint32_t u_raw) {
  const float g = raw16_to_float(g_raw & 0xffffu, AT{});
  const float u = raw16_to_float(u_raw & 0xffffu, AT{});
  const float s = raw16_to_float(to_raw16(g / (1.0f + expf(-g)), AT{}), AT{});
  return s * u;
}

// Logical column -> storage index of a bias permuted with marlin_permute_bias
// (reference sm70_marlin_bias.cuh:18-25; marlin_utils.py:279-314).
__device__ __forceinline__ int bias_storage_index(int col) {
  // scale_perm_single: storage p holds logical col 2*(p/8) + {0,1,8,9,16,17,24,25}[p%8]
  // within each 32-column group; this is its inverse.
  const int lc = col & 31;
  const int i = lc >> 3;           // which of {0,1},{8,9},{16,17},{24,25} pair-group
  const int r = lc & 7;            // 2*(p/8) + j  with j in {0,1}
  const int p = (r >> 1) * 8 + i * 2 + (r & 1);
  return (col & ~31) + p;
}

}  // namespace mmi
