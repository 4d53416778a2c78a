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

#include "mxgg_internal.h"

namespace mxgg {

enum { kModeRceil = 0, kModeFloor = 1 };

// Largest group table a token-axis cast stages in LDS (the ABI's expert limit).
constexpr int kMaxGroups = 1024;

// amax16 = max over the block of (bf16 bits & 0x7FFF).  For non-negative bf16
// bit patterns integer order equals magnitude order and every NaN pattern
// (> 0x7F80) sorts above +Inf, so an integer max propagates NaN.
template <int MODE>
__device__ __forceinline__ uint32_t e8m0_from_amax16(uint32_t amax16) {
  const uint32_t ex = amax16 >> 7;
  const uint32_t mant = amax16 & 0x7Fu;
  // RCEIL: amax/448 <= 2^j  <=>  amax <= 1.75 * 2^(j+8).  With amax = 1.m *
  // 2^(ex-127): j = ex-135 when 1.m <= 1.75 (mant <= 0x60), else ex-134; b = j + 127.
  // FLOOR: b = ex - 8.  Both clamp at 0; Inf gives 254 (RCEIL) / 247 (FLOOR),
  // NaN 255.  Written as selects: no branch per block.
  const int nb = (int)ex - 8 + (MODE == kModeRceil && mant > 0x60u ? 1 : 0);
  const uint32_t finite = (uint32_t)(nb < 0 ? 0 : (nb > 254 ? 254 : nb));
  const uint32_t special = mant ? 255u : (MODE == kModeRceil ? 254u : 247u);
  return ex == 255u ? special : finite;
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

__device__ __forceinline__ uint32_t amax16_of_word(uint32_t w) {
  const uint32_t lo = w & 0x7FFFu, hi = (w >> 16) & 0x7FFFu;
  return lo > hi ? lo : hi;
}

// Max over the four lanes of a quad, through DPP quad permutations [1,0,3,2]
// and [2,3,0,1] (VALU only, no LDS round trip).  Every lane of the quad must
// be active.
__device__ __forceinline__ uint32_t quad_max(uint32_t x) {
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0xB1, 0xF, 0xF, false));
  return max(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x4E, 0xF, 0xF, false));
}

// Streaming (nontemporal) 8-byte store of payload bytes that this kernel does
// not read back.
__device__ __forceinline__ void store_stream(uint8_t* p, uint2 v) {
  __builtin_nontemporal_store(u32x2{v.x, v.y}, reinterpret_cast<u32x2*>(p));
}

// Lane-wise max of two pairs of 16-bit integers (v_pk_max_u16).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// |x| bit patterns of the two bf16 of a word, still packed.
__device__ __forceinline__ uint32_t abs_bf16x2(uint32_t w) { return w & 0x7FFF7FFFu; }

// amax16 of the eight bf16 values of a 16-byte chunk.
__device__ __forceinline__ uint32_t amax16_of_chunk(const uint4& v) {
  const uint32_t m = pk_max_u16(pk_max_u16(abs_bf16x2(v.x), abs_bf16x2(v.y)),
                                pk_max_u16(abs_bf16x2(v.z), abs_bf16x2(v.w)));
  return max(m & 0xFFFFu, m >> 16);
}

// Payload bytes of four values (bf16 values widened to float) of a block with
// scale byte b, for a block without NaN (b != 255): scale, clamp, convert.
template <int MODE, bool SW>
__device__ __forceinline__ uint32_t encode4_finite(float x0, float x1, float x2, float x3,
                                                   uint32_t b) {
  int e = payload_exponent<MODE>(b);
  asm("" : "+v"(e));  // one exponent per block: keep it out of the per-value code
  const float y0 = __builtin_fminf(__builtin_fmaxf(__builtin_ldexpf(x0, e), -448.0f), 448.0f);
  const float y1 = __builtin_fminf(__builtin_fmaxf(__builtin_ldexpf(x1, e), -448.0f), 448.0f);
  const float y2 = __builtin_fminf(__builtin_fmaxf(__builtin_ldexpf(x2, e), -448.0f), 448.0f);
  const float y3 = __builtin_fminf(__builtin_fmaxf(__builtin_ldexpf(x3, e), -448.0f), 448.0f);
  if (SW)
    return e4m3_encode_sw(y0) | (e4m3_encode_sw(y1) << 8) | (e4m3_encode_sw(y2) << 16) |
           (e4m3_encode_sw(y3) << 24);
  const uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y0, y1, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y2, y3, (int)w, true);
}

// The same for any block, NaN blocks included (b == 255 in both modes exactly
// when the block holds a NaN): NaN values keep their sign as code 0x7F | sign,
// and FLOOR divides a NaN block by +inf.
template <int MODE, bool SW>
__device__ __forceinline__ uint32_t encode4_any(float x0, float x1, float x2, float x3,
                                                uint32_t b) {
  const int e = payload_exponent<MODE>(b);
  const bool floor_nan = MODE == kModeFloor && b == 255u;
  float y[4] = {x0, x1, x2, x3};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    y[i] = floor_nan ? floor_nan_block_value(y[i]) : scale_and_clamp(y[i], e);
  return e4m3_pack4<SW>(y[0], y[1], y[2], y[3]);
}

// Compile-time choice: ANY = some block of the wave needs the full encoder
// (needs_full_encoder; callers test that once per wave with __any, so the
// common case has no per-lane branch and no NaN or Inf handling).
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ uint32_t encode4_sel(float x0, float x1, float x2, float x3,
                                                uint32_t b) {
  return ANY ? encode4_any<MODE, SW>(x0, x1, x2, x3, b)
             : encode4_finite<MODE, SW>(x0, x1, x2, x3, b);
}

// Two bf16 packed in a word, widened to float.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Scale bytes whose blocks the short encoder must not take (callers reduce
// this over the wave and pick ANY = true when any lane has one): NaN blocks
// (255) in every configuration, and for RCEIL with the hardware converter also
// blocks holding an infinity (254, which no finite amax reaches: the largest
// finite bf16 gives 247), since v_cvt_scalef32_pk_fp8_bf16 does not clamp and
// would turn inf into the NaN code instead of 448.
template <int MODE, bool SW>
__device__ __forceinline__ bool needs_full_encoder(uint32_t b) {
  return (MODE == kModeRceil && !SW) ? b >= 254u : b == 255u;
}

// Payload bytes of the four bf16 values in words w0 (bytes 0, 1) and w1
// (bytes 2, 3) of a block with scale byte b.  RCEIL through the hardware
// converter: v_cvt_scalef32_pk_fp8_bf16 divides a bf16 pair by the scale
// 2^(b-127) and rounds to nearest even, which is exactly x * 2^(127-b) rounded
// as the f32 path rounds it.  RCEIL picks b so that amax <= 448 * 2^(b-127),
// so no value of a finite block needs the clamp; b == 0 means a multiplier of
// 1.  Checked bit for bit against the f32 path over every bf16 pattern and
// scale byte; the GPU cast tests repeat that through the oracle.
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ uint32_t encode4_words(uint32_t w0, uint32_t w1, uint32_t b) {
  if constexpr (MODE == kModeRceil && !SW && !ANY) {
    typedef short i16x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const float s = b == 0u ? 1.0f : __uint_as_float(b << 23);
    i16x2 o = {0, 0};
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(bf16x2, w0), s, false);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(bf16x2, w1), s, true);
    return __builtin_bit_cast(uint32_t, o);
  } else {
    return encode4_sel<MODE, SW, ANY>(bf16_lo(w0), bf16_hi(w0), bf16_lo(w1), bf16_hi(w1), b);
  }
}

// Word of bf16 values lo16(a) | lo16(b) << 16 (HI: the high halves).
template <bool HI>
__device__ __forceinline__ uint32_t pair_halves(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, HI ? 0x07060302u : 0x05040100u);
}

// max of the two 16-bit halves of a, and of b, packed: low half from a.
__device__ __forceinline__ uint32_t half_max_pair(uint32_t a, uint32_t b) {
  return pk_max_u16(pair_halves<false>(a, b), pair_halves<true>(a, b));
}

// Payload bytes of the eight bf16 values of a chunk under block byte b
// (ANY: see encode4_sel).
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ uint2 encode_chunk8(const uint4& v, uint32_t b) {
  return make_uint2(encode4_words<MODE, SW, ANY>(v.x, v.y, b),
                    encode4_words<MODE, SW, ANY>(v.z, v.w, b));
}

// Sixteen scale bytes b[0..15] (one per word) written to p..p+15 as one
// 16-byte store at any byte alignment: gfx9 global stores take unaligned
// addresses (the compiler lowers a 16-byte memcpy to one global_store_dwordx4
// for this target), where byte stores would cost 16 store instructions.
__device__ __forceinline__ void store_scale_bytes16(uint8_t* p, const uint32_t (&b)[16]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = b[4 * k] | (b[4 * k + 1] << 8) | (b[4 * k + 2] << 16) | (b[4 * k + 3] << 24);
  __builtin_memcpy(p, w, 16);
}

// Two floats rounded to bf16 (round to nearest even, v_cvt_pk_bf16_f32) and
// packed into one word, `lo` in bits 0-15.  Finite and infinite values round as
// torch's float -> bfloat16 conversion does; a NaN stays a NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// a / b for finite a and 1 <= b < 2^126, from the hardware reciprocal and one
// Newton step on the residual (fma): the classic correction that returns the
// correctly rounded quotient except in rare near-tie cases.  Outside that
// domain (b = inf, or a reciprocal below the normal range, which v_rcp_f32
// flushes to zero) callers divide with the compiler's IEEE division.
__device__ __forceinline__ float div_nr_finite(float a, float b) {
  const float r = __builtin_amdgcn_rcpf(b);
  const float q = a * r;
  return __builtin_fmaf(__builtin_fmaf(-q, b, a), r, q);
}

// exp(x) for |x| <= 88, where neither overflow nor underflow can occur.
// Cody-Waite reduction: x * log2(e) = n + f, with log2(e) split into a float
// and the float of the remainder, n = rint, 2^f from v_exp_f32 and n put back
// by ldexp.  These are the steps and the order of operations that the
// device library's expf compiles to on gfx950 for such x, so the bits agree;
// that function also tests x against its overflow and underflow bounds,
// which this one leaves out.
__device__ __forceinline__ float exp_moderate(float x) {
  // no contraction: ph must be rounded before n is subtracted from it
#pragma clang fp contract(off)
  constexpr float kLog2eHi = 0x1.715476p+0f;
  constexpr float kLog2eLo = 0x1.4ae0bep-26f;
  const float ph = x * kLog2eHi;
  const float pl = __builtin_fmaf(x, kLog2eLo, __builtin_fmaf(x, kLog2eHi, -ph));
  const float n = __builtin_rintf(ph);
  return __builtin_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), (int)n);
}

// bf16 bit pattern of 87.0: |g| at or below it keeps exp(-g) finite and
// 1 + exp(-g) below 2^126 (e^87 = 6.1e37 < 8.5e37), the domain of
// exp_moderate and div_nr_finite.
constexpr uint32_t kBf16Moderate = 0x42AEu;

// SwiGLU of the two bf16 values of a word of gate and of up:
// a = bf16(bf16(g / (1 + exp(-g))) * u), packed (torch's eager bf16
// F.silu(gate) * up).  Shared by the standalone SwiGLU kernels and the
// gate+up GEMM epilogue, so both give the same bits.
// MOD: |g| <= 87 (kBf16Moderate) for both values, so exp(-g) needs no range
// tests and the quotient can come from the corrected reciprocal; otherwise
// IEEE division, exact for every input.
template <bool MOD>
__device__ __forceinline__ uint32_t swiglu_a_word(uint32_t gw, uint32_t uw) {
  const float g0 = bf16_lo(gw), g1 = bf16_hi(gw);
  const uint32_t sw =
      MOD ? pack_bf16x2(div_nr_finite(g0, 1.0f + exp_moderate(-g0)),
                        div_nr_finite(g1, 1.0f + exp_moderate(-g1)))
          : pack_bf16x2(g0 / (1.0f + expf(-g0)), g1 / (1.0f + expf(-g1)));
  return pack_bf16x2(bf16_lo(sw) * bf16_lo(uw), bf16_hi(sw) * bf16_hi(uw));
}

// SwiGLU of a 16-byte chunk (eight values).  Activations almost always have
// |gate| <= 87: a chunk whose gate values are all in that range in every lane
// of the wave takes the math without range tests (one vote, no per-lane
// branch).  Callers run it with the whole wave active.
__device__ __forceinline__ uint4 swiglu_a_chunk(const uint4& g, const uint4& u) {
  const uint32_t gm = pk_max_u16(pk_max_u16(abs_bf16x2(g.x), abs_bf16x2(g.y)),
                                 pk_max_u16(abs_bf16x2(g.z), abs_bf16x2(g.w)));
  if (__all(max(gm & 0xFFFFu, gm >> 16) <= kBf16Moderate))
    return make_uint4(swiglu_a_word<true>(g.x, u.x), swiglu_a_word<true>(g.y, u.y),
                      swiglu_a_word<true>(g.z, u.z), swiglu_a_word<true>(g.w, u.w));
  return make_uint4(swiglu_a_word<false>(g.x, u.x), swiglu_a_word<false>(g.y, u.y),
                    swiglu_a_word<false>(g.z, u.z), swiglu_a_word<false>(g.w, u.w));
}

// Group tables of the token-axis casts, staged in LDS by every workgroup:
//   ends_s[g] : end of group g clamped to [0, rows]
//   pend_s[g] : padded cumulative end (every group rounded up to 32 tokens),
//               as written by the padded-ends kernel
// Callers synchronise the workgroup before reading the tables.
__device__ __forceinline__ void stage_group_tables(const int32_t* __restrict__ ends,
                                                   const int32_t* __restrict__ ends_pad, int E,
                                                   int64_t rows, int32_t* ends_s,
                                                   int32_t* pend_s) {
  for (int g = threadIdx.x; g < E; g += blockDim.x) pend_s[g] = ends_pad[g];
  monotone_ends_to_lds(ends, E, rows, ends_s);
}

// bf16(float(v_i) * sc) for the eight bf16 values of a 16-byte chunk (RNE).
__device__ __forceinline__ uint4 scale_chunk(const uint4& v, float sc) {
  return make_uint4(pack_bf16x2(bf16_lo(v.x) * sc, bf16_hi(v.x) * sc),
                    pack_bf16x2(bf16_lo(v.y) * sc, bf16_hi(v.y) * sc),
                    pack_bf16x2(bf16_lo(v.z) * sc, bf16_hi(v.z) * sc),
                    pack_bf16x2(bf16_lo(v.w) * sc, bf16_hi(v.w) * sc));
}

// Padded token position P, the first of a run of `run` positions (run divides
// 32, P a multiple of run, so the run never straddles two groups), to the
// first real token tok0 and the number of real tokens ntok in the run.
// Positions past a group's real tokens and past the padded total map to none.
__device__ __forceinline__ void padded_run_tokens(int64_t P, int run, const int32_t* ends_s,
                                                  const int32_t* pend_s, int E, int64_t& tok0,
                                                  int& ntok) {
  tok0 = 0;
  ntok = 0;
  int lo = 0, hi = E;  // first group whose padded end is > P
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((int64_t)pend_s[mid] > P) hi = mid; else lo = mid + 1;
  }
  if (lo < E) {
    const int64_t pstart = lo > 0 ? pend_s[lo - 1] : 0;
    const int64_t gstart = lo > 0 ? ends_s[lo - 1] : 0;
    const int64_t gend = ends_s[lo];
    tok0 = gstart + (P - pstart);
    const int64_t n = gend - tok0;  // negative when the clamped start exceeds the end
    ntok = n <= 0 ? 0 : (n >= run ? run : (int)n);
  }
}

}  // namespace mxgg
