// Device-side MXFP8 helpers shared by the quantisation and GEMM kernels.
//
// E8M0 scale rules (one byte b per 32-element block, value 2^(b-127)):
//   RCEIL : b = clamp(ceil(log2(amax / 448)), -127, 127) + 127, NaN block -> 0xFF
//           (torchao recipe "mxfp8_rceil", selected by the reference's trainer
//            integration at port_mxfp8.py:178,207-213)
//   FLOOR : b = clamp(floor(log2(amax)) - 8, -127, 128) + 127, NaN block -> 0xFF
//           (OCP MX v1.0 "emax of e4m3 = 8" rule)
// Payload: RNE_e4m3fn(clamp(x * mult, -448, 448)) with
//   RCEIL : mult = 1 if b == 0 else 2^(127-b)
//   FLOOR : mult = 1 / max(2^(b-127), 2^-126)   (b == 255 divides by +inf)
// NaN inputs keep their sign: code 0x7F | sign.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxgg {

enum { kModeRceil = 0, kModeFloor = 1 };

// amax16 = max over the block of (bf16 bits & 0x7FFF).  For non-negative bf16
// bit patterns integer order equals magnitude order and every NaN pattern
// (> 0x7F80) sorts above +Inf, so an integer max propagates NaN.
template <int MODE>
__device__ __forceinline__ uint32_t e8m0_from_amax16(uint32_t amax16) {
  const uint32_t ex = amax16 >> 7;
  const uint32_t mant = amax16 & 0x7Fu;
  if (ex == 255u) return mant ? 255u : (MODE == kModeRceil ? 254u : 247u);
  if (MODE == kModeRceil) {
    // amax/448 <= 2^j  <=>  amax <= 1.75 * 2^(j+8).  With amax = 1.m * 2^(ex-127):
    // j = ex-135 when 1.m <= 1.75 (mant <= 0x60), else ex-134.  b = j + 127.
    int b = (int)ex - 8 + (mant > 0x60u ? 1 : 0);
    return (uint32_t)(b < 0 ? 0 : (b > 254 ? 254 : b));
  } else {
    int b = (int)ex - 8;
    return (uint32_t)(b < 0 ? 0 : b);
  }
}

// Power-of-two exponent applied to the payload for a given scale byte.
template <int MODE>
__device__ __forceinline__ int payload_exponent(uint32_t b) {
  if (MODE == kModeRceil) return b == 0u ? 0 : 127 - (int)b;
  return 127 - (int)(b < 1u ? 1u : b);  // FLOOR, b <= 254 (255 handled apart)
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// x * 2^e, then clamp to [-448, 448] keeping NaN.
__device__ __forceinline__ float scale_and_clamp(float x, int e) {
  float y = __builtin_ldexpf(x, e);
  float c = __builtin_fminf(__builtin_fmaxf(y, -448.0f), 448.0f);
  return (y != y) ? y : c;
}

// FLOOR mode, NaN block (b = 0xFF): x / +inf -> +-0 for finite x, NaN otherwise.
__device__ __forceinline__ float floor_nan_block_value(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7F800000u) != 0x7F800000u) return __uint_as_float(u & 0x80000000u);
  if ((u & 0x7FFFFFFFu) == 0x7F800000u) return __uint_as_float(0x7FC00000u);  // inf/inf
  return x;
}

// Bit-level RNE encoder to OCP e4m3fn for |y| <= 448 or NaN.
__device__ __forceinline__ uint32_t e4m3_encode_sw(float y) {
  const uint32_t u = __float_as_uint(y);
  const uint32_t s = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return s | 0x7Fu;
  if (a < 0x3C800000u) {  // |y| < 2^-6: subnormal grid, step 2^-9
    const float t = __uint_as_float(a) * 512.0f;
    return s | (uint32_t)__builtin_rintf(t);
  }
  // Normal: keep 3 mantissa bits with round-half-even at bit 20, rebias 127 -> 7.
  const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
  return s | (r - 960u);
}

// Encode four already clamped floats into four e4m3 bytes (little endian).
template <bool SW>
__device__ __forceinline__ uint32_t e4m3_pack4(float a, float b, float c, float d) {
  if (SW) {
    return e4m3_encode_sw(a) | (e4m3_encode_sw(b) << 8) | (e4m3_encode_sw(c) << 16) |
           (e4m3_encode_sw(d) << 24);
  }
  uint32_t w = 0;
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)w, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  // NaN inputs: force the canonical code 0x7F with the input's sign.
  const float v[4] = {a, b, c, d};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (v[i] != v[i]) {
      const uint32_t code = 0x7Fu | ((__float_as_uint(v[i]) >> 24) & 0x80u);
      w = (w & ~(0xFFu << (8 * i))) | (code << (8 * i));
    }
  }
  return w;
}

// Quantise two bf16 packed in one 32-bit word with block byte b, giving
// two payload floats ready for packing.
template <int MODE>
__device__ __forceinline__ void bf16x2_to_scaled(uint32_t w, uint32_t b, int e, float& lo,
                                                 float& hi) {
  const float x0 = bf16_bits_to_f32(w & 0xFFFFu);
  const float x1 = bf16_bits_to_f32(w >> 16);
  if (MODE == kModeFloor && b == 255u) {
    lo = floor_nan_block_value(x0);
    hi = floor_nan_block_value(x1);
  } else {
    lo = scale_and_clamp(x0, e);
    hi = scale_and_clamp(x1, e);
  }
}

__device__ __forceinline__ uint32_t amax16_of_word(uint32_t w) {
  const uint32_t lo = w & 0x7FFFu, hi = (w >> 16) & 0x7FFFu;
  return lo > hi ? lo : hi;
}

}  // namespace mxgg
