// SwiGLU activation of the expert FFN fused with the MXFP8 casts around it.
//
// The gate+up projection writes h = [gate | up] in bf16.  The down projection
// needs a = SiLU(gate) * up cast along its features (row-wise, 1x32 blocks);
// the backward pass needs, from h and the gradient da of a:
//   dh = [d_gate | d_up]   cast row-wise      (dX = dh . W_gate_up)
//   dh                     cast along tokens  (dW_gate_up = dh^T . X)
//   a                      cast along tokens  (dW_down = dY^T . a)
// Each of the two kernels reads its bf16 inputs once and writes every cast
// directly; no bf16 intermediate goes through HBM.
//
// Arithmetic is torch's eager bf16 semantics for the same expression
// (F.silu(gate) * up with autograd), so the fused path equals the unfused one
// (bit for bit on the GPU in the tests; for gates with |g| <= 87 the
// quotients below come from a corrected reciprocal, which matches the IEEE
// quotient except in rare near-tie cases, beyond that from IEEE division, and
// bf16 rounding is the hardware round-to-nearest-even):
//   s      = bf16(g / (1 + exp(-g)))                 (silu, fp32 inside)
//   a      = bf16(s * u)
//   d_up   = bf16(da * s)
//   d_gate = bf16(bf16(da * u) * sig * (1 + g * (1 - sig))),  sig = 1 / (1 + exp(-g))
// The reference computes the same activation eagerly in bf16
// (e2e_bench.py:56-61 forward, :85-100 backward).
#include <algorithm>

#include "mx_device.h"
#include "mxgg_internal.h"

namespace mxgg {
namespace {

struct ActWord {
  uint32_t a, dg, du;  // two packed bf16 results each
};

// exp(-g) and a / b; MOD: |g| <= 87 (kBf16Moderate) holds for every value, so
// exp needs no overflow or underflow tests and the quotient can come from
// the corrected reciprocal; otherwise expf and IEEE division, exact for
// every input.
template <bool MOD>
__device__ __forceinline__ float exp_neg(float g) {
  return MOD ? exp_moderate(-g) : expf(-g);
}
template <bool MOD>
__device__ __forceinline__ float quot(float a, float b) {
  return MOD ? div_nr_finite(a, b) : a / b;
}

template <bool MOD>
__device__ __forceinline__ float dsilu_term(float ds, float g, float ex) {
  const float sig = quot<MOD>(1.0f, 1.0f + ex);
  return ds * sig * (1.0f + g * (1.0f - sig));
}

// a, d_gate and d_up for the two values of a word of gate, up and grad_a.
template <bool MOD>
__device__ __forceinline__ ActWord swiglu_bwd_word(uint32_t gw, uint32_t uw, uint32_t dw) {
  const float g0 = bf16_lo(gw), g1 = bf16_hi(gw);
  const float u0 = bf16_lo(uw), u1 = bf16_hi(uw);
  const float d0 = bf16_lo(dw), d1 = bf16_hi(dw);
  const float e0 = exp_neg<MOD>(g0), e1 = exp_neg<MOD>(g1);
  const uint32_t sw = pack_bf16x2(quot<MOD>(g0, 1.0f + e0),
                                  quot<MOD>(g1, 1.0f + e1));  // s = bf16(silu(g))
  const uint32_t dsw = pack_bf16x2(d0 * u0, d1 * u1);                   // bf16(grad_a * up)
  const float s0 = bf16_lo(sw), s1 = bf16_hi(sw);
  ActWord r;
  r.a = pack_bf16x2(s0 * u0, s1 * u1);
  r.du = pack_bf16x2(d0 * s0, d1 * s1);
  r.dg = pack_bf16x2(dsilu_term<MOD>(bf16_lo(dsw), g0, e0),
                     dsilu_term<MOD>(bf16_hi(dsw), g1, e1));
  return r;
}

// a, d_gate and d_up of a lane's 16 token rows x 4 features, in place of
// gate, up and grad_a, one token at a time (interleaving all 32 exp/div
// chains would need far more registers than this streaming kernel can hold).
// Activations almost always have |gate| <= 87: a token row whose gate values
// are all in that range in every lane of the wave takes the math without
// range tests (one vote per row, no per-lane branch).
__device__ __forceinline__ void swiglu_bwd_rows(uint2 (&A)[16], uint2 (&DG)[16], uint2 (&DU)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t gm = pk_max_u16(abs_bf16x2(A[i].x), abs_bf16x2(A[i].y));
    ActWord r0, r1;
    if (__all(max(gm & 0xFFFFu, gm >> 16) <= kBf16Moderate)) {
      r0 = swiglu_bwd_word<true>(A[i].x, DG[i].x, DU[i].x);
      r1 = swiglu_bwd_word<true>(A[i].y, DG[i].y, DU[i].y);
    } else {
      r0 = swiglu_bwd_word<false>(A[i].x, DG[i].x, DU[i].x);
      r1 = swiglu_bwd_word<false>(A[i].y, DG[i].y, DU[i].y);
    }
    A[i] = make_uint2(r0.a, r1.a);
    DG[i] = make_uint2(r0.dg, r1.dg);
    DU[i] = make_uint2(r0.du, r1.du);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ---------------------------------------------------------------------------
// Forward: a = SiLU(gate) * up, cast row-wise.  Same shape as the dim0 cast:
// a lane owns one 8-feature chunk of a row (gate and up chunk loaded as one
// 16-byte vector each), a quad holds one 32-feature block, a wave 4 rows per
// trip, a workgroup 16 rows.
// ---------------------------------------------------------------------------
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ void swiglu_dim0_store(const uint4 (&a)[4], const uint32_t (&b)[4],
                                                  uint16_t* a_out, int64_t lda, uint8_t* q,
                                                  int64_t ldq, uint8_t* s, int64_t s_row,
                                                  int64_t s_blk, int64_t r0, int64_t rows, int cc,
                                                  bool col_ok, int lane) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t r = r0 + k;
    const uint2 o = encode_chunk8<MODE, SW, ANY>(a[k], b[k]);
    if (col_ok && r < rows) {
      *reinterpret_cast<uint2*>(q + r * ldq + (int64_t)cc * 8) = o;
      if (a_out != nullptr) *reinterpret_cast<uint4*>(a_out + r * lda + (int64_t)cc * 8) = a[k];
    }
  }
  // the quad's scale bytes of rows r0 .. r0+3: contiguous in block-major
  // storage (one 4-byte store), else one byte per row
  if (col_ok && (lane & 3) == 0) {
    uint8_t* sp = s + (int64_t)(cc >> 2) * s_blk;
    if (s_row == 1 && r0 + 4 <= rows && (reinterpret_cast<uintptr_t>(sp + r0) & 3u) == 0) {
      *reinterpret_cast<uint32_t*>(sp + r0) = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (r0 + k < rows) sp[(r0 + k) * s_row] = (uint8_t)b[k];
    }
  }
}

template <int MODE, bool SW>
__global__ __launch_bounds__(256) void k_swiglu_dim0(
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up, int64_t ldh, int64_t rows,
    int cols8, uint16_t* __restrict__ a_out, int64_t lda, uint8_t* __restrict__ q, int64_t ldq,
    uint8_t* __restrict__ s, int64_t s_row, int64_t s_blk) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int cc = blockIdx.x * 64 + lane;
  const bool col_ok = cc < cols8;  // whole quads share col_ok (cols8 % 4 == 0)
  for (int64_t r0 = (int64_t)blockIdx.y * 16 + wave * 4; r0 < rows; r0 += (int64_t)gridDim.y * 16) {
    uint4 g[4], u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t r = r0 + k;
      if (col_ok && r < rows) {
        g[k] = *reinterpret_cast<const uint4*>(gate + r * ldh + (int64_t)cc * 8);
        u[k] = *reinterpret_cast<const uint4*>(up + r * ldh + (int64_t)cc * 8);
      } else {
        g[k] = make_uint4(0, 0, 0, 0);
        u[k] = make_uint4(0, 0, 0, 0);
      }
    }
    uint4 a[4];
    uint32_t b[4];
    bool nan = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a[k] = swiglu_a_chunk(g[k], u[k]);
      uint32_t am = amax16_of_chunk(a[k]);
      am = quad_max(am);
      b[k] = e8m0_from_amax16<MODE>(am);
      nan |= needs_full_encoder<MODE, SW>(b[k]);
    }
    if (__any(nan))
      swiglu_dim0_store<MODE, SW, true>(a, b, a_out, lda, q, ldq, s, s_row, s_blk, r0, rows, cc,
                                        col_ok, lane);
    else
      swiglu_dim0_store<MODE, SW, false>(a, b, a_out, lda, q, ldq, s, s_row, s_blk, r0, rows, cc,
                                         col_ok, lane);
  }
}

// ---------------------------------------------------------------------------
// Backward.  A workgroup covers 128 padded token positions x 128 features of
// a (so 2 x 128 features of h and dh); wave w takes positions 32w .. 32w+31,
// exactly one 32-token scale block.  Lane (tg = lane % 2, fg = lane / 2) owns
// 16 positions (16 tg ..) and 4 features (4 fg ..): it loads 16 token rows of
// gate, up and da as 8-byte vectors (32 lanes read 256 contiguous bytes of a
// row), computes a, d_gate and d_up in registers (in place of the inputs),
// and emits
//   row-wise casts of d_gate / d_up: a 32-feature block is the eight lanes
//     of one 16-lane row with the same tg (amax combined with DPP rotations
//     by 2, 4 and 8 within the row); a wave's store covers whole 128-byte
//     lines of two token rows;
//   token-axis casts of a, d_gate, d_up: a 32-token block is the two lanes
//     tg = 0, 1 (one DPP swap), 16 payload bytes per feature, so the four
//     waves write 128 contiguous bytes of every output row.
// (Measured at C5's shape: 3.2 TB/s with 32 positions x 64 features per
// workgroup, whose row-wise lines were split between two workgroups, 3.8 TB/s
// so.  Streaming stores pay off for the whole-line row-wise stores only.)
// Padded positions map to tokens as in the token-axis cast; a run of 16 never
// straddles a group because groups start on multiples of 32.
// ---------------------------------------------------------------------------
struct SwigluBwdArgs {
  const uint16_t* gate;
  const uint16_t* up;
  const uint16_t* da;
  const int32_t* ends;      // nullptr = one group of `rows` tokens
  const int32_t* ends_pad;
  uint8_t* dq;              // row-wise cast of [d_gate | d_up]: [rows, 2 cols]
  uint8_t* ds;
  uint8_t* dqt;             // token-axis cast of [d_gate | d_up]: [2 cols, cap]
  uint8_t* dst;
  uint8_t* aqt;             // token-axis cast of a: [cols, cap]
  uint8_t* ast;
  uint16_t* dh;             // optional bf16 [d_gate | d_up]: [rows, 2 cols]
  int64_t ldh, ldda, rows, cap;
  int64_t lddq, ds_row, ds_blk;
  int64_t lddqt, dst_row, dst_blk;
  int64_t ldaqt, ast_row, ast_blk;
  int64_t lddh;
  int32_t cols, E;
};

// Token-axis cast of the lane's 4 features x 16 positions held in v[0..15]:
// feature j goes to row j of `qrow` (16 payload bytes; qrow already points at
// column P of the lane's first feature row).  ANY: some block of the wave
// needs the full encoder (decided once per wave, so the common case runs the short
// encoder without per-lane branches).
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ void token_axis_payload(const uint2 (&v)[16], const uint32_t (&bytes)[4],
                                                   uint8_t* qrow, int64_t ldqt, bool out_ok) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // feature j of positions 4k .. 4k+3, paired into two bf16 words
      const uint32_t w0 = (j >> 1) == 0 ? v[4 * k].x : v[4 * k].y;
      const uint32_t w1 = (j >> 1) == 0 ? v[4 * k + 1].x : v[4 * k + 1].y;
      const uint32_t w2 = (j >> 1) == 0 ? v[4 * k + 2].x : v[4 * k + 2].y;
      const uint32_t w3 = (j >> 1) == 0 ? v[4 * k + 3].x : v[4 * k + 3].y;
      const uint32_t p0 = (j & 1) ? pair_halves<true>(w0, w1) : pair_halves<false>(w0, w1);
      const uint32_t p1 = (j & 1) ? pair_halves<true>(w2, w3) : pair_halves<false>(w2, w3);
      o[k] = encode4_words<MODE, SW, ANY>(p0, p1, bytes[j]);
    }
    if (out_ok) *reinterpret_cast<uint4*>(qrow + j * ldqt) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Max of the two lanes of a pair (DPP quad permutation [1,0,3,2]).
__device__ __forceinline__ uint32_t pair_max_u16x2(uint32_t x) {
  return pk_max_u16(x, (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0xB1, 0xF, 0xF, false));
}

template <int MODE, bool SW>
__device__ __forceinline__ void emit_token_axis(const uint2 (&v)[16], uint8_t* qrow, int64_t ldqt,
                                                uint8_t* srow, int64_t st_row, bool out_ok,
                                                bool scale_lane) {
  // amax of both features of a word at once (packed 16-bit max), combined
  // over the two lanes of the 32-token block.
  uint32_t mx = 0, my = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    mx = pk_max_u16(mx, abs_bf16x2(v[i].x));
    my = pk_max_u16(my, abs_bf16x2(v[i].y));
  }
  mx = pair_max_u16x2(mx);
  my = pair_max_u16x2(my);
  uint32_t bytes[4];
  bytes[0] = e8m0_from_amax16<MODE>(mx & 0xFFFFu);
  bytes[1] = e8m0_from_amax16<MODE>(mx >> 16);
  bytes[2] = e8m0_from_amax16<MODE>(my & 0xFFFFu);
  bytes[3] = e8m0_from_amax16<MODE>(my >> 16);
  const bool nan = needs_full_encoder<MODE, SW>(bytes[0]) ||
                   needs_full_encoder<MODE, SW>(bytes[1]) ||
                   needs_full_encoder<MODE, SW>(bytes[2]) || needs_full_encoder<MODE, SW>(bytes[3]);
  if (__any(nan))
    token_axis_payload<MODE, SW, true>(v, bytes, qrow, ldqt, out_ok);
  else
    token_axis_payload<MODE, SW, false>(v, bytes, qrow, ldqt, out_ok);
  if (out_ok && scale_lane) {
    if (st_row == 1 && (reinterpret_cast<uintptr_t>(srow) & 3u) == 0) {
      *reinterpret_cast<uint32_t*>(srow) =
          bytes[0] | (bytes[1] << 8) | (bytes[2] << 16) | (bytes[3] << 24);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) srow[(int64_t)j * st_row] = (uint8_t)bytes[j];
    }
  }
}

// Row-wise cast of 4 features x 16 tokens (chunk v[i] of token i) into qrow
// (row of the first token, already offset to the lane's column); the eight
// lanes of a 32-feature block share amax.
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ void row_wise_payload(const uint2 (&v)[16], const uint32_t (&bytes)[16],
                                                 uint8_t* qrow, int64_t ldq, int ntok) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t o = encode4_words<MODE, SW, ANY>(v[i].x, v[i].y, bytes[i]);
    if (i < ntok) __builtin_nontemporal_store(o, reinterpret_cast<uint32_t*>(qrow + i * ldq));
  }
}

// Writes n <= 16 scale bytes b[j] at p[j * stride], as one 16-byte store when
// all sixteen are contiguous (at any alignment: a run of 16 tokens starts
// wherever its group does).
__device__ __forceinline__ void store_scale16(uint8_t* p, int64_t stride, const uint32_t (&b)[16],
                                              int n) {
  if (stride == 1 && n == 16) {
    store_scale_bytes16(p, b);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < n) p[(int64_t)j * stride] = (uint8_t)b[j];
  }
}

template <int MODE, bool SW>
__device__ __forceinline__ void emit_row_wise(const uint2 (&v)[16], uint8_t* qrow, int64_t ldq,
                                              uint8_t* srow, int64_t s_row, int ntok,
                                              bool scale_lane) {
  // amax of each token's 4 features, two tokens packed per shuffle, combined
  // over the eight lanes of the 32-feature block.
  uint32_t bytes[16];
  bool nan = false;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t m0 = pk_max_u16(abs_bf16x2(v[2 * t].x), abs_bf16x2(v[2 * t].y));
    const uint32_t m1 = pk_max_u16(abs_bf16x2(v[2 * t + 1].x), abs_bf16x2(v[2 * t + 1].y));
    uint32_t m = half_max_pair(m0, m1);
    // the block's eight lanes are those of one 16-lane row with the same
    // parity: rotations by 2, 4 and 8 within the row reach all of them
    m = pk_max_u16(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x122, 0xF, 0xF, false));
    m = pk_max_u16(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x124, 0xF, 0xF, false));
    m = pk_max_u16(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x128, 0xF, 0xF, false));
    bytes[2 * t] = e8m0_from_amax16<MODE>(m & 0xFFFFu);
    bytes[2 * t + 1] = e8m0_from_amax16<MODE>(m >> 16);
    nan |= needs_full_encoder<MODE, SW>(bytes[2 * t]) ||
           needs_full_encoder<MODE, SW>(bytes[2 * t + 1]);
  }
  if (__any(nan))
    row_wise_payload<MODE, SW, true>(v, bytes, qrow, ldq, ntok);
  else
    row_wise_payload<MODE, SW, false>(v, bytes, qrow, ldq, ntok);
  if (scale_lane && ntok > 0) store_scale16(srow, s_row, bytes, ntok);
}

// Optional bf16 copy of 16 token rows x 4 features (dh may be null).
__device__ __forceinline__ void store_bf16_rows(const uint2 (&v)[16], uint16_t* dh, int64_t off,
                                                int64_t ld, int ntok) {
  if (dh == nullptr) return;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < ntok) *reinterpret_cast<uint2*>(dh + off + i * ld) = v[i];
}

// 16 token rows of three inputs stay in registers: two waves per SIMD.
template <int MODE, bool SW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_swiglu_bwd(
    const SwigluBwdArgs p) {
  __shared__ int32_t ends_s[kMaxGroups];
  __shared__ int32_t pend_s[kMaxGroups];
  const int lane = threadIdx.x & 63;
  const int tg = lane & 1, fg = lane >> 1;
  const uint32_t nfb = ((uint32_t)p.cols + 127u) / 128u;
  const uint32_t fb = blockIdx.x % nfb, pb = blockIdx.x / nfb;
  const int64_t P = (int64_t)pb * 128 + (threadIdx.x >> 6) * 32 + 16 * tg;
  const int f = (int)fb * 128 + 4 * fg;

  int64_t tok0 = 0;
  int ntok = 0;
  if (p.ends != nullptr) {
    stage_group_tables(p.ends, p.ends_pad, p.E, p.rows, ends_s, pend_s);
    __syncthreads();
    padded_run_tokens(P, 16, ends_s, pend_s, p.E, tok0, ntok);
  } else {
    tok0 = P;
    const int64_t n = p.rows - P;
    ntok = n <= 0 ? 0 : (n >= 16 ? 16 : (int)n);
  }
  if (f >= p.cols) ntok = 0;

  const uint16_t* gp = p.gate + tok0 * p.ldh + f;
  const uint16_t* upp = p.up + tok0 * p.ldh + f;
  const uint16_t* dp = p.da + tok0 * p.ldda + f;
  // gate, up and da are loaded into A, DG, DU and replaced there by a,
  // d_gate and d_up
  uint2 A[16], DG[16], DU[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    A[i] = DG[i] = DU[i] = make_uint2(0, 0);
    if (i < ntok) {
      A[i] = *reinterpret_cast<const uint2*>(gp + i * p.ldh);
      DG[i] = *reinterpret_cast<const uint2*>(upp + i * p.ldh);
      DU[i] = *reinterpret_cast<const uint2*>(dp + i * p.ldda);
    }
  }
  swiglu_bwd_rows(A, DG, DU);

  const int64_t cols = p.cols;
  store_bf16_rows(DG, p.dh, tok0 * p.lddh + f, p.lddh, ntok);
  store_bf16_rows(DU, p.dh, tok0 * p.lddh + cols + f, p.lddh, ntok);

  const bool row_scale_lane = (fg & 7) == 0;
  uint8_t* qrow = p.dq + tok0 * p.lddq + f;
  uint8_t* srow = p.ds + tok0 * p.ds_row;
  emit_row_wise<MODE, SW>(DG, qrow, p.lddq, srow + (int64_t)(f >> 5) * p.ds_blk, p.ds_row, ntok,
                          row_scale_lane);
  emit_row_wise<MODE, SW>(DU, qrow + cols, p.lddq, srow + ((cols + f) >> 5) * p.ds_blk, p.ds_row,
                          ntok, row_scale_lane);

  const bool out_ok = f < p.cols && P < p.cap;
  const bool tok_scale_lane = tg == 0;
  const int64_t sblk = P >> 5;
  emit_token_axis<MODE, SW>(A, p.aqt + (int64_t)f * p.ldaqt + P, p.ldaqt,
                            p.ast + (int64_t)f * p.ast_row + sblk * p.ast_blk, p.ast_row, out_ok,
                            tok_scale_lane);
  emit_token_axis<MODE, SW>(DG, p.dqt + (int64_t)f * p.lddqt + P, p.lddqt,
                            p.dst + (int64_t)f * p.dst_row + sblk * p.dst_blk, p.dst_row, out_ok,
                            tok_scale_lane);
  emit_token_axis<MODE, SW>(DU, p.dqt + (cols + f) * p.lddqt + P, p.lddqt,
                            p.dst + (cols + f) * p.dst_row + sblk * p.dst_blk, p.dst_row, out_ok,
                            tok_scale_lane);
}

template <int MODE, bool SW>
hipError_t swiglu_dim0_impl(const uint16_t* gate, const uint16_t* up, int64_t ldh, int64_t rows,
                            int64_t cols, uint16_t* a_out, int64_t lda, uint8_t* q, int64_t ldq,
                            uint8_t* s, int64_t s_row, int64_t s_blk, hipStream_t stream) {
  const int cols8 = (int)(cols / 8);
  dim3 grid((cols8 + 63) / 64, (unsigned)std::min<int64_t>((rows + 15) / 16, 65535));
  hipLaunchKernelGGL((k_swiglu_dim0<MODE, SW>), grid, dim3(256), 0, stream, gate, up, ldh, rows,
                     cols8, a_out, lda, q, ldq, s, s_row, s_blk);
  return hipGetLastError();
}

template <int MODE, bool SW>
hipError_t swiglu_bwd_impl(const SwigluBwdArgs& p, hipStream_t stream) {
  dim3 grid((unsigned)(((p.cap + 127) / 128) * ((p.cols + 127) / 128)));
  hipLaunchKernelGGL((k_swiglu_bwd<MODE, SW>), grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_swiglu_quant_dim0(const uint16_t* gate, const uint16_t* up, int64_t ldh,
                                    int64_t rows, int64_t cols, uint16_t* a_out, int64_t lda,
                                    uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, int layout,
                                    int mode, hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const bool sw = (mode & kCvtSoftwareFlag) != 0;
  const int m = mode & 0xFF;
  const int64_t s_row = layout == MXGG_SCALES_BLOCK_MAJOR ? 1 : lds;
  const int64_t s_blk = layout == MXGG_SCALES_BLOCK_MAJOR ? lds : 1;
#define MXGG_SWIGLU0(MODE, SWF) \
  swiglu_dim0_impl<MODE, SWF>(gate, up, ldh, rows, cols, a_out, lda, q, ldq, s, s_row, s_blk, stream)
  if (m == kModeRceil) return sw ? MXGG_SWIGLU0(kModeRceil, true) : MXGG_SWIGLU0(kModeRceil, false);
  return sw ? MXGG_SWIGLU0(kModeFloor, true) : MXGG_SWIGLU0(kModeFloor, false);
#undef MXGG_SWIGLU0
}

hipError_t launch_swiglu_bwd_quant(const SwigluBwdLaunch& l, hipStream_t stream) {
  if (l.cols == 0 || l.cap == 0) return hipSuccess;
  if (l.group_ends != nullptr) {
    const hipError_t err = launch_pad_ends(l.group_ends, l.num_groups, l.rows, l.group_ends_pad,
                                           stream);
    if (err != hipSuccess) return err;
  }
  const bool bm = l.layout == MXGG_SCALES_BLOCK_MAJOR;
  SwigluBwdArgs p;
  p.gate = l.gate;
  p.up = l.up;
  p.da = l.da;
  p.ends = l.group_ends;
  p.ends_pad = l.group_ends_pad;
  p.dq = l.dq;
  p.ds = l.ds;
  p.dqt = l.dqt;
  p.dst = l.dst;
  p.aqt = l.aqt;
  p.ast = l.ast;
  p.dh = l.dh;
  p.ldh = l.ldh;
  p.ldda = l.ldda;
  p.rows = l.rows;
  p.cap = l.cap;
  p.lddq = l.lddq;
  p.ds_row = bm ? 1 : l.ldds;
  p.ds_blk = bm ? l.ldds : 1;
  p.lddqt = l.lddqt;
  p.dst_row = bm ? 1 : l.lddst;
  p.dst_blk = bm ? l.lddst : 1;
  p.ldaqt = l.ldaqt;
  p.ast_row = bm ? 1 : l.ldast;
  p.ast_blk = bm ? l.ldast : 1;
  p.lddh = l.lddh;
  p.cols = (int32_t)l.cols;
  p.E = (int32_t)(l.group_ends != nullptr ? l.num_groups : 1);
  const bool sw = (l.mode & kCvtSoftwareFlag) != 0;
  const int m = l.mode & 0xFF;
  if (m == kModeRceil)
    return sw ? swiglu_bwd_impl<kModeRceil, true>(p, stream)
              : swiglu_bwd_impl<kModeRceil, false>(p, stream);
  return sw ? swiglu_bwd_impl<kModeFloor, true>(p, stream)
            : swiglu_bwd_impl<kModeFloor, false>(p, stream);
}

}  // namespace mxgg
