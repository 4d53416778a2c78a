// Internal declarations shared by the HIP translation units of libmxgg.so.
// gfx950 (CDNA4) only: wave64, scaled MFMA (f8f6f4), 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mxgg.h"

namespace mxgg {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Flag OR-ed into scale_mode: use the bit-level software e4m3 encoder instead
// of v_cvt_pk_fp8_f32.  Both must give identical bytes; the flag exists so the
// GPU tests can check the hardware convert against an independent encoder.
constexpr int kCvtSoftwareFlag = 0x100;

// Group ends as every kernel of the library reads them: m[g] = the running
// maximum of ends[0..g], clamped to [0, rows]; group g covers rows
// [m[g-1], m[g]) (m[-1] = 0).  Monotone input is used as given; a decreasing
// entry makes its group empty instead of letting it overlap an earlier one, so
// no row belongs to two groups and the group sizes sum to at most `rows`.
// Called by every thread of the block; ends in the device array `ends`, the
// result in LDS `m[E]`; ends with a barrier.
__device__ __forceinline__ void monotone_ends_to_lds(const int32_t* __restrict__ ends, int E,
                                                     int64_t rows, int32_t* m) {
  for (int g = threadIdx.x; g < E; g += blockDim.x) {
    const int32_t e = ends[g];
    m[g] = e < 0 ? 0 : (e > rows ? (int32_t)rows : e);
  }
  __syncthreads();
  int bad = 0;
  for (int g = threadIdx.x + 1; g < E; g += blockDim.x) bad |= m[g] < m[g - 1];
  // Well-formed ends (the usual case) cost one vote; others a serial pass.
  if (__syncthreads_or(bad)) {
    if (threadIdx.x == 0)
      for (int g = 1; g < E; ++g) m[g] = m[g] > m[g - 1] ? m[g] : m[g - 1];
    __syncthreads();
  }
}

// Error reporting (capi.hip).
int set_error(int status, const char* fmt, ...);

// Number of compute units of the current device (cached per device).
int device_cu_count();

// ---------------------------------------------------------------------------
// Launchers (implemented in quant.hip / gemm.hip).  Arguments are validated by
// the C-ABI layer before these are called.
// ---------------------------------------------------------------------------
hipError_t launch_quant_dim0(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                             uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, int layout,
                             int mode, hipStream_t stream);

hipError_t launch_quant_dim1(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                             const int32_t* group_ends, int64_t num_groups,
                             int64_t rows_pad_cap, uint8_t* qt, int64_t ldqt, uint8_t* st,
                             int64_t ldst, int layout, int32_t* group_ends_pad, int mode,
                             hipStream_t stream);

// Both casts from one read: row-wise (q, s: as launch_quant_dim0, rows inside
// groups) and token-axis (qt, st: as launch_quant_dim1).  q == nullptr gives the
// token-axis cast alone.
hipError_t launch_quant_dual(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                             const int32_t* group_ends, int64_t num_groups,
                             int64_t rows_pad_cap, uint8_t* q, int64_t ldq, uint8_t* s,
                             int64_t lds, uint8_t* qt, int64_t ldqt, uint8_t* st, int64_t ldst,
                             int layout, int32_t* group_ends_pad, int mode, hipStream_t stream);

// The dual cast of rows gathered from token order: row r of the input is row
// src[r] / topk of x (zero for src[r] < 0), times row_scale[src[r]] (rounded to
// bf16) when row_scale is given; rows = rows of the routed layout.
hipError_t launch_gather_quant_dual(const uint16_t* x, int64_t xrows, int64_t ldx,
                                    const int32_t* src, int topk, const float* row_scale,
                                    int64_t rows, int64_t cols, const int32_t* group_ends,
                                    int64_t num_groups, int64_t rows_pad_cap, uint8_t* q,
                                    int64_t ldq, uint8_t* s, int64_t lds, uint8_t* qt,
                                    int64_t ldqt, uint8_t* st, int64_t ldst, int layout,
                                    int32_t* group_ends_pad, int mode, hipStream_t stream);

// The row-wise cast of rows gathered from token order (row r = row
// src[r] / topk of x, zero for src[r] < 0); rows = rows of the routed layout.
hipError_t launch_gather_quant_dim0(const uint16_t* x, int64_t xrows, int64_t ldx,
                                    const int32_t* src, int topk, int64_t rows, int64_t cols,
                                    uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, int layout,
                                    int mode, hipStream_t stream);

// Token routing (route.hip).
hipError_t launch_route_plan(const int32_t* idx, int64_t n, int E, int pad, int64_t cap,
                             int32_t* perm, int32_t* src, int32_t* ends, int32_t* counts,
                             hipStream_t stream);
// The same plan over route_plan_blocks(n) workgroups, with a workspace of
// route_plan_blocks(n) * E int32 (no initialisation).
int64_t route_plan_blocks(int64_t n);
hipError_t launch_route_plan_blocks(const int32_t* idx, int64_t n, int E, int pad, int64_t cap,
                                    int32_t* perm, int32_t* src, int32_t* ends, int32_t* counts,
                                    int32_t* ws, hipStream_t stream);
hipError_t launch_gather_rows(const uint16_t* x, int64_t ldx, int64_t xrows, const int32_t* src,
                              int topk, const float* row_scale, int64_t rows, int64_t cols,
                              uint16_t* out, int64_t ldo, hipStream_t stream);
hipError_t launch_combine(const uint16_t* y, int64_t ldy, int64_t yrows, const int32_t* perm,
                          const float* scores, int64_t tokens, int topk, int64_t cols, uint16_t* out,
                          int64_t ldo, hipStream_t stream);
hipError_t launch_combine_score_grad(const uint16_t* dout, int64_t ldd, const uint16_t* y,
                                     int64_t ldy, int64_t yrows, const int32_t* perm,
                                     int64_t tokens, int topk, int64_t cols, float* dscore,
                                     hipStream_t stream);

// Group-offset utilities (groups.hip).
hipError_t launch_offs_to_ends(const int32_t* offs, int64_t E, int64_t tokens, int kind,
                               int32_t* ends, hipStream_t stream);
hipError_t launch_zero_tail(uint8_t* out, int64_t rows, int64_t row_bytes, int64_t ld_bytes,
                            const int32_t* ends, int64_t E, hipStream_t stream);

// Padded cumulative group ends of the token-axis casts (one workgroup).
hipError_t launch_pad_ends(const int32_t* group_ends, int64_t num_groups, int64_t rows,
                           int32_t* group_ends_pad, hipStream_t stream);

// SwiGLU fused with its casts (swiglu.hip).
hipError_t launch_swiglu_quant_dim0(const uint16_t* gate, const uint16_t* up, int64_t ldh,
                                    int64_t rows, int64_t cols, uint16_t* a_out, int64_t lda,
                                    uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, int layout,
                                    int mode, hipStream_t stream);

struct SwigluBwdLaunch {
  const uint16_t* gate;
  const uint16_t* up;
  const uint16_t* da;
  const int32_t* group_ends;  // nullptr = one group
  int32_t* group_ends_pad;
  uint8_t* dq;   // row-wise cast of [d_gate | d_up]
  uint8_t* ds;
  uint8_t* dqt;  // token-axis cast of [d_gate | d_up]
  uint8_t* dst;
  uint8_t* aqt;  // token-axis cast of a
  uint8_t* ast;
  uint16_t* dh;  // optional bf16 [d_gate | d_up]
  int64_t ldh, ldda, rows, cols, num_groups, cap;
  int64_t lddq, ldds, lddqt, lddst, ldaqt, ldast, lddh;
  int layout, mode;
};
hipError_t launch_swiglu_bwd_quant(const SwigluBwdLaunch& l, hipStream_t stream);

hipError_t launch_scales_to_block_major(const uint8_t* src, int64_t batch, int64_t rows,
                                        int64_t nblk, int64_t sb, int64_t lds, uint8_t* dst,
                                        int64_t db, int64_t ldd, hipStream_t stream);

struct FwdArgs {
  const uint8_t* a;
  const uint8_t* as;   // block-major [K/32][ldas]
  const uint8_t* w;
  const uint8_t* ws;   // per expert block-major [K/32][ldws]
  const int32_t* group_ends;  // nullptr = one group of M rows
  void* out;
  int64_t lda, ldas, w_gstride, ldw, ws_gstride, ldws, ldo;
  int32_t M, N, K, E;
  int32_t out_f32;
  int32_t scaled;
  // Optional workspace of fwd_split_workspace_bytes(): the tiles of a last,
  // sparse round of tiles are then split along K over the idle CUs.
  float* split_ws;
  // Fused SwiGLU output (swiglu_mode = MXGG_SCALE_RCEIL / _FLOOR, -1 = off):
  // w holds [gate; up] (N = 2F rows), and the kernel writes the row-wise
  // MXFP8 cast of a = SiLU(gate) * up: payload aq [M, F] (row stride ldaq
  // bytes), scale byte (m, b) at as_out[m * as_row + b * as_blk].  `out` is
  // then either nullptr or the bf16 [gate | up] rows h [M, 2F] (row stride ldo
  // elements, 16-byte aligned rows).
  int32_t swiglu_mode;
  uint8_t* aq;
  uint8_t* as_out;
  int64_t ldaq, as_row, as_blk;
};
hipError_t launch_grouped_fwd(const FwdArgs& args, hipStream_t stream);
int64_t fwd_split_workspace_bytes();
// The library's own per-device scratch for the forward split (device address
// of the current device's copy, nullptr if the symbol lookup fails) and its size.
void* noalloc_scratch();
int64_t noalloc_scratch_bytes();

struct WgradArgs {
  const uint8_t* go;   // [N, M] token-contiguous
  const uint8_t* gos;  // block-major [M/32][ldgos]
  const uint8_t* ia;   // [K, M]
  const uint8_t* ias;  // block-major [M/32][ldias]
  const int32_t* group_ends;
  void* dw;            // dW[g][n][k] at element g * ldw_e + n * ldw_n + k
  int64_t ldgo, ldgos, ldia, ldias;
  int64_t ldw_e, ldw_n;  // elements; N * K and K for a contiguous [E, N, K]
  int32_t M, N, K, E;
  int32_t split;       // tokens per split-K chunk (multiple of 128), 0 = whole groups
  int32_t out_f32;
  int32_t scaled;
  // With split > 0: workspace of wgrad_split_workspace_bytes() for the fp32
  // partials, added in chunk order by a second kernel (deterministic, any
  // output dtype); nullptr = fp32 atomics into the zeroed output.
  float* split_ws;
};
hipError_t launch_grouped_wgrad(const WgradArgs& args, hipStream_t stream);
int64_t wgrad_split_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t E, int64_t split);

}  // namespace mxgg
