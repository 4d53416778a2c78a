/*
 * mxgg.h — C ABI of libmxgg.so, the MI355X (gfx950) MXFP8 grouped-GEMM library.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element
 * counts and leading dimensions, launches asynchronously on the caller's HIP
 * stream (passed as `void*`, i.e. a `hipStream_t`), never allocates or frees
 * device memory, never synchronises the host, and returns an `mxgg_status`.
 * No C++ exception crosses the boundary.  On error a human readable reason is
 * available from `mxgg_last_error()` (thread local).
 *
 * Data formats (OCP Microscaling v1.0):
 *   payload  : float8 e4m3fn, one byte per element (torch.float8_e4m3fn)
 *   scale    : E8M0, one byte b per block of 32 payload elements along the
 *              contraction dimension, meaning 2^(b-127); 0xFF is NaN
 *   bf16     : bfloat16, two bytes per element
 * Leading dimensions (`ld*`) are in ELEMENTS of the array they describe.
 * Groups ("experts") are described by `group_ends[num_groups]`, int32,
 * cumulative end offsets (group g covers [group_ends[g-1], group_ends[g]),
 * group 0 starts at 0) — the convention of torch._grouped_mm and of the
 * reference's callers (e2e_bench.py:42, wgrad_fused.py:64).  Empty groups are
 * allowed.  `group_ends` lives in device memory and is read only on the GPU.
 * Ends that decrease or leave [0, rows] are read as their running maximum
 * clamped to [0, rows] (see mxgg_offs_to_group_ends), so groups never overlap.
 */
#ifndef MXGG_H
#define MXGG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXGG_ABI_VERSION 13

typedef enum mxgg_status {
  MXGG_OK = 0,
  MXGG_ERR_INVALID_ARGUMENT = 1, /* null pointer, unknown enum value          */
  MXGG_ERR_SHAPE = 2,            /* negative / inconsistent sizes, K % 32 != 0 */
  MXGG_ERR_ALIGNMENT = 3,        /* pointer or leading dimension misaligned    */
  MXGG_ERR_UNSUPPORTED = 4,      /* size outside the supported envelope        */
  MXGG_ERR_DEVICE = 5,           /* no HIP device / not gfx950                 */
  MXGG_ERR_LAUNCH = 6            /* kernel launch reported an error            */
} mxgg_status;

typedef enum mxgg_scale_mode {
  MXGG_SCALE_RCEIL = 0, /* b = ceil(log2(amax/448)) + 127   (recipe "mxfp8_rceil") */
  MXGG_SCALE_FLOOR = 1  /* b = floor(log2(amax)) - 8 + 127  (OCP MX v1.0 rule)      */
} mxgg_scale_mode;

typedef enum mxgg_out_dtype {
  MXGG_OUT_BF16 = 0,
  MXGG_OUT_F32 = 1
} mxgg_out_dtype;

/*
 * Memory layout of an E8M0 scale matrix that is logically [rows, nblk]
 * (nblk = contraction length / 32):
 *   ROW_MAJOR   : byte (r, b) at s[r * ld + b]   (the reference's [M, K//32]
 *                 uint8 tensors, fused_fwd.py:182-183)
 *   BLOCK_MAJOR : byte (r, b) at s[b * ld + r]   (one row of bytes per
 *                 32-deep k-block; what the GEMM kernels consume, so a stage
 *                 of 256 rows reads its scales as one contiguous run)
 */
typedef enum mxgg_scale_layout {
  MXGG_SCALES_ROW_MAJOR = 0,
  MXGG_SCALES_BLOCK_MAJOR = 1
} mxgg_scale_layout;

/*
 * How a caller's `offs` vector describes the expert groups (mxgg_offs_to_group_ends).
 *   ENDS  : cumulative token ends (torch._grouped_mm convention; the reference's
 *           layer step, e2e_bench.py:42,117)
 *   SIZES : tokens per group (the reference's wgrad_fused documentation,
 *           wgrad_fused.py:37, and its wgrad benchmark, bench_wgrad_dsv3.py:52)
 *   AUTO  : SIZES when the entries add up to exactly `tokens` and the last entry
 *           is below `tokens`, ENDS otherwise
 */
typedef enum mxgg_offs_kind {
  MXGG_OFFS_ENDS = 0,
  MXGG_OFFS_SIZES = 1,
  MXGG_OFFS_AUTO = 2
} mxgg_offs_kind;

/* ABI version of the loaded library (MXGG_ABI_VERSION at build time). */
int mxgg_abi_version(void);

/* Static string naming a status code. */
const char* mxgg_status_string(int status);

/* Detailed message for the last non-OK status returned on this thread. */
const char* mxgg_last_error(void);

/*
 * Row-wise MXFP8 cast: 1x32 blocks along the last (contiguous) dimension.
 *   x      : bf16 [rows, cols], row stride ldx
 *   q      : e4m3 [rows, cols], row stride ldq
 *   scales : E8M0, logically [rows, cols/32], in `scale_layout` with stride lds
 * cols % 32 == 0.  Payload = RNE_e4m3(clamp(x * 2^(127-b), -448, 448)).
 * Replaces torchao's triton_to_mxfp8_dim0 (called by the reference's trainer
 * path, port_mxfp8.py:43-49) and the eager `.to(torch.float8_e4m3fn)` casts on
 * the forward path (e2e_bench.py:35-40,60, fused_fwd.py:274-275).
 */
int mxgg_quant_dim0(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                    void* q, int64_t ldq, void* scales, int64_t lds, int scale_layout,
                    int scale_mode, void* stream);

/*
 * Token-axis (column-wise) MXFP8 cast with per-group block restart, written
 * transposed: 1x32 blocks run along `rows` (tokens) and never straddle a group
 * boundary; each group is zero-padded to a multiple of 32 tokens.
 *   x              : bf16 [rows, cols], row stride ldx
 *   group_ends     : int32 [num_groups] cumulative token ends (device), or NULL
 *                    for a single group covering all rows
 *   rows_pad_cap   : number of padded token columns the outputs can hold; must
 *                    be >= round_up(rows + 31*num_groups, 32) (NULL groups: round_up(rows,32))
 *   qt             : e4m3 [cols, rows_pad_cap], row stride ldqt
 *   scales_t       : E8M0, logically [cols, rows_pad_cap/32], in
 *                    `scale_layout` with stride ldst
 *   group_ends_pad : int32 [num_groups] padded cumulative ends (device, written)
 *                    or NULL when group_ends is NULL
 * Columns past the padded total are written as zero payload with the scale of an
 * all-zero block (byte 0).
 * Replaces torchao's triton_to_mxfp8_dim1 (port_mxfp8.py:43) plus the
 * transpose-and-stack copies of wgrad_fused.py:48-62 / e2e_bench.py:114-126.
 */
int mxgg_quant_dim1(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                    const int32_t* group_ends, int64_t num_groups,
                    int64_t rows_pad_cap, void* qt, int64_t ldqt,
                    void* scales_t, int64_t ldst, int scale_layout,
                    int32_t* group_ends_pad, int scale_mode, void* stream);

/*
 * Both casts of one bf16 matrix from a single read: the row-wise cast of
 * mxgg_quant_dim0 (q, scales) and the token-axis cast of mxgg_quant_dim1
 * (qt, scales_t, group_ends_pad), with the argument rules of each.  For
 * operands that a training step contracts both ways: the layer input X and the
 * output gradient dY (forward / dgrad vs wgrad), and expert weights viewed as
 * [E*N, K] with group_ends = N, 2N, .. (forward vs dgrad).  cols % 32 == 0.
 * Row-wise rows are written for the rows inside the groups (all rows when
 * group_ends is NULL).  scale_layout applies to both scale outputs.
 * Replaces the pair of torchao casts triton_to_mxfp8_dim0 / _dim1 that the
 * reference's trainer path runs on the same tensor (port_mxfp8.py:43-49).
 */
int mxgg_quant_dual(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                    const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap, void* q,
                    int64_t ldq, void* scales, int64_t lds, void* qt, int64_t ldqt,
                    void* scales_t, int64_t ldst, int scale_layout, int32_t* group_ends_pad,
                    int scale_mode, void* stream);

/*
 * SwiGLU activation fused with the row-wise MXFP8 cast of its output:
 *   a = bf16(bf16(silu(gate)) * up),  silu(g) = g / (1 + exp(-g)) in fp32
 * (torch's eager bf16 result of F.silu(gate) * up).
 *   gate, up : bf16 [rows, cols], common row stride ldh (e.g. the two column
 *              halves of the gate+up projection output h = [gate | up])
 *   q, scales: the cast of a, as mxgg_quant_dim0 writes it
 *   a_out    : optional bf16 [rows, cols] copy of a (row stride lda), or NULL
 * cols % 32 == 0.  Replaces the eager `silu(hg) * hu` and `.to(float8)` of the
 * reference's layer step (e2e_bench.py:56-61).
 */
int mxgg_swiglu_quant_dim0(const void* gate, const void* up, int64_t ldh, int64_t rows,
                           int64_t cols, void* a_out, int64_t lda, void* q, int64_t ldq,
                           void* scales, int64_t lds, int scale_layout, int scale_mode,
                           void* stream);

/*
 * SwiGLU backward fused with the three casts the backward GEMMs consume.
 * From gate, up (bf16 [rows, cols], stride ldh) and grad_a = dL/da (bf16
 * [rows, cols], stride ldga), with s = bf16(silu(gate)), sig = sigmoid(gate):
 *   d_up   = bf16(grad_a * s)
 *   d_gate = bf16(bf16(grad_a * up) * sig * (1 + gate * (1 - sig)))
 *   a      = bf16(s * up)
 * (torch's eager bf16 autograd of F.silu(gate) * up), and writes
 *   dh_q, dh_scales      : row-wise cast of dh = [d_gate | d_up], [rows, 2*cols]
 *                          (as mxgg_quant_dim0) — the dX operand
 *   dh_qt, dh_scales_t   : token-axis cast of dh, transposed, [2*cols, rows_pad_cap]
 *                          (as mxgg_quant_dim1) — the dW_gate_up operand
 *   a_qt, a_scales_t     : token-axis cast of a, transposed, [cols, rows_pad_cap]
 *                          — the dW_down operand
 *   group_ends_pad       : padded group ends (as mxgg_quant_dim1)
 *   dh_out               : optional bf16 dh [rows, 2*cols] (stride lddh), or NULL
 * group_ends / num_groups / rows_pad_cap as for mxgg_quant_dim1.  Rows past the
 * last group end get no row-wise output.  scale_layout applies to all three
 * scale outputs.  cols % 32 == 0.  Replaces the reference's eager SiLU
 * backward (e2e_bench.py:85-100) and the casts of its wgrad operands
 * (e2e_bench.py:114-126).
 */
int mxgg_swiglu_bwd_quant(const void* gate, const void* up, int64_t ldh, const void* grad_a,
                          int64_t ldga, int64_t rows, int64_t cols, const int32_t* group_ends,
                          int64_t num_groups, int64_t rows_pad_cap, void* dh_q, int64_t lddq,
                          void* dh_scales, int64_t ldds, void* dh_qt, int64_t lddqt,
                          void* dh_scales_t, int64_t lddst, void* a_qt, int64_t ldaqt,
                          void* a_scales_t, int64_t ldast, int32_t* group_ends_pad, void* dh_out,
                          int64_t lddh, int scale_layout, int scale_mode, void* stream);

/*
 * Re-lay E8M0 scales from ROW_MAJOR to BLOCK_MAJOR, batched:
 *   dst[b][k][r] = src[b][r][k]   for b < batch, r < rows, k < nblk
 * src batch stride / row stride: src_bstride / lds; dst: dst_bstride / ldd.
 * For callers holding the reference's row-major [M, K/32] / [E, N, K/32]
 * uint8 scales; the library's own casts can emit BLOCK_MAJOR directly.
 * (No reference counterpart: the reference's kernels read row-major scales
 * inside the GEMM, fused_fwd.py:112-123.)
 */
int mxgg_scales_to_block_major(const void* src, int64_t batch, int64_t rows, int64_t nblk,
                               int64_t src_bstride, int64_t lds, void* dst,
                               int64_t dst_bstride, int64_t ldd, void* stream);

/*
 * Group ends from a caller's `offs` (int32 [num_groups], device) read as
 * `offs_kind`: group_ends = offs (ENDS) or its inclusive prefix sum (SIZES,
 * saturated to int32), chosen on the device for AUTO with `tokens` the token
 * count of the operands.  One workgroup, no host sync; group_ends may not
 * alias offs.  1 <= num_groups <= 1024.
 * Replaces nothing in the reference, whose wgrad entry points read only
 * offs.shape[0] and split M // E tokens per expert (wgrad_fused.py:45-47); it
 * lets the same call sites (wgrad_fused.py:37 sizes, e2e_bench.py:117 ends)
 * honour unequal groups.
 *
 * Every kernel of this library reads group ends by one rule: m[g] = the
 * running maximum of group_ends[0..g] clamped to [0, rows]; group g covers
 * [m[g-1], m[g]) (m[-1] = 0).  Non-decreasing ends are used as given; a
 * decreasing entry makes its group empty, so no row belongs to two groups.
 */
int mxgg_offs_to_group_ends(const int32_t* offs, int64_t num_groups, int64_t tokens,
                            int offs_kind, int32_t* group_ends, void* stream);

/*
 * Zero the rows of a row-major matrix that lie past the last group end
 * (rows r >= m[num_groups-1] under the rule above), which no grouped GEMM
 * writes: out holds `rows` rows of `row_bytes` bytes with stride `ld_bytes`;
 * out, row_bytes and ld_bytes are multiples of 16.  The end is read on the
 * device.  For callers that hand the whole matrix on, e.g. as an input
 * gradient to autograd (the reference has no counterpart: its groups always
 * cover every row, fused_fwd.py:47-48).
 */
int mxgg_zero_rows_past_groups(void* out, int64_t rows, int64_t row_bytes, int64_t ld_bytes,
                               const int32_t* group_ends, int64_t num_groups, void* stream);

/*
 * Forward grouped GEMM  out[rows of g] = A[rows of g] . W[g]^T  (fp32 accumulate).
 *   a        : e4m3 [M, K], row stride lda
 *   a_scales : E8M0 BLOCK_MAJOR [K/32][ldas], ldas >= M       (or NULL)
 *   w        : e4m3 [E, N, K]: expert g at w + g*w_group_stride, row stride ldw
 *              (experts may overlap or interleave: e.g. column blocks of one
 *              transposed weight matrix, as for dX = dY . W)
 *   w_scales : E8M0 BLOCK_MAJOR, expert g at + g*ws_group_stride: [K/32][ldws],
 *              ldws >= N                                       (or NULL)
 *   Scale strides and bases are multiples of 4 bytes, and a block-major array
 *   of nblk block-rows holding `rows` rows must be readable for
 *   (nblk-1)*ld + round_up(rows, 4) bytes from its base (per expert for w).
 *   group_ends : int32 [num_groups] (device) or NULL for one group of M rows
 *   out      : [M, N] bf16 or f32 (out_dtype), row stride ldo; base aligned
 *              to 4 elements and ldo a multiple of 4 (any N: columns past the
 *              last whole 4-element group are stored one by one)
 * a_scales and w_scales are both given or both NULL (NULL = every scale 1.0,
 * E8M0 byte 0x7F).  K % 32 == 0.  Rows past the last group end are untouched.
 * a and w are 16-byte aligned, lda and ldw multiples of 16 and at most 2^23,
 * each operand spans less than 2 GiB; strides that are multiples of 128 let
 * every load fetch whole cache lines (the fast case).
 * Replaces fused_grouped_fwd (fused_fwd.py:172-229) + its kernel
 * (fused_fwd.py:18-167), and fwd_ge (fwd_final.py:121-131) with num_groups=1.
 */
int mxgg_grouped_fwd(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                     const void* w, int64_t w_group_stride, int64_t ldw,
                     const void* w_scales, int64_t ws_group_stride, int64_t ldws,
                     const int32_t* group_ends, int64_t num_groups,
                     int64_t M, int64_t N, int64_t K,
                     void* out, int64_t ldo, int out_dtype, void* stream);

/*
 * Forward grouped GEMM of the gate+up projection fused with SwiGLU and the
 * row-wise MXFP8 cast of its result, for the forward-only (inference) pass:
 *   h[rows of g] = A[rows of g] . W[g]^T      (fp32 accumulate, rounded to bf16)
 *   a = bf16(bf16(silu(h[:, :F])) * h[:, F:])  (as mxgg_swiglu_quant_dim0)
 * and writes only the cast of a: payload q [M, F] e4m3 (row stride ldq) and
 * E8M0 scales, logically [M, F/32], in `scale_layout` with stride lds.
 *   w : [E, 2F, K] e4m3, gate rows 0..F-1 then up rows F..2F-1 of each expert
 *       (the fused gate+up weight), with w_scales as for mxgg_grouped_fwd
 * Every other argument as mxgg_grouped_fwd (N = 2F).  F % 128 == 0.  The
 * result equals mxgg_grouped_fwd (bf16 out) followed by
 * mxgg_swiglu_quant_dim0 on the rows inside the groups; rows past the last
 * group end are not written.  bf16 h is never written to memory.
 * Replaces the reference's forward layer step gate/up GEMMs, eager
 * `silu(hg) * hu` and `.to(float8)` (e2e_bench.py:56-61).
 */
int mxgg_grouped_fwd_swiglu_quant(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                                  const void* w, int64_t w_group_stride, int64_t ldw,
                                  const void* w_scales, int64_t ws_group_stride, int64_t ldws,
                                  const int32_t* group_ends, int64_t num_groups, int64_t M,
                                  int64_t F, int64_t K, void* q, int64_t ldq, void* scales,
                                  int64_t lds, int scale_layout, int scale_mode, void* stream);

/*
 * mxgg_grouped_fwd_swiglu_quant for the training forward: also writes the
 * bf16 gate+up projection h [M, 2F] (gate columns 0..F-1, up columns F..2F-1;
 * row stride ldh elements, ldh >= 2F, ldh % 8 == 0, h 16-byte aligned) that
 * the SwiGLU backward (mxgg_swiglu_bwd_quant) re-reads.  h equals
 * mxgg_grouped_fwd's bf16 output bit for bit and q / scales equal
 * mxgg_grouped_fwd_swiglu_quant's, on the rows inside the groups; rows past
 * the last group end are not written.  Saves the standalone SwiGLU cast's
 * re-read of h.
 * Replaces the reference's training layer step gate/up GEMMs, eager
 * `silu(hg) * hu` (whose inputs autograd keeps for the backward) and
 * `.to(float8)` (e2e_bench.py:56-61).
 */
int mxgg_grouped_fwd_swiglu_quant_keep_h(const void* a, int64_t lda, const void* a_scales,
                                         int64_t ldas, const void* w, int64_t w_group_stride,
                                         int64_t ldw, const void* w_scales,
                                         int64_t ws_group_stride, int64_t ldws,
                                         const int32_t* group_ends, int64_t num_groups, int64_t M,
                                         int64_t F, int64_t K, void* h, int64_t ldh, void* q,
                                         int64_t ldq, void* scales, int64_t lds, int scale_layout,
                                         int scale_mode, void* stream);

/*
 * mxgg_grouped_fwd with a caller-owned workspace of at least
 * mxgg_grouped_fwd_workspace_bytes() bytes (16-byte aligned; contents need no
 * initialisation and are scratch after the call).  When the tiles of the
 * last round would leave at least half of the compute units idle (and for
 * launches with fewer tiles than compute units), those tiles are cut along K
 * into up to 16 ranges over the idle units; their fp32 partial tiles go to the
 * workspace and a second kernel on the same stream adds them in a fixed order
 * and writes the output.  Deterministic; results can differ from
 * mxgg_grouped_fwd in the last bit of those tiles (fp32 summation order).
 * Replaces the same reference interface as mxgg_grouped_fwd
 * (fused_fwd.py:172-229); the reference has no counterpart of the workspace.
 * Calls that share a workspace must be ordered on one stream.
 */
int64_t mxgg_grouped_fwd_workspace_bytes(void);
int mxgg_grouped_fwd_split(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                           const void* w, int64_t w_group_stride, int64_t ldw,
                           const void* w_scales, int64_t ws_group_stride, int64_t ldws,
                           const int32_t* group_ends, int64_t num_groups,
                           int64_t M, int64_t N, int64_t K,
                           void* out, int64_t ldo, int out_dtype,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mxgg_grouped_fwd_split without a workspace argument and without any
 * allocation: the split partials go to scratch memory the library holds per
 * device (a static device array of 16 KB + 256 x 256 KB = 64 MiB + 16 KiB,
 * reserved on every device the library runs on until the process ends).
 * Same arguments, results and rules as mxgg_grouped_fwd_split; calls no
 * hipMalloc / hipFree.  Returns MXGG_ERR_UNSUPPORTED on a device whose
 * persistent grid needs more than 256 partials (more than 256 compute units).
 * Every call on one device shares that scratch, which keeps the last call's
 * contents: calls that overlap in time on one device (different streams, or
 * graph replays running concurrently) race; calls ordered on one stream are
 * safe.  Nothing in it needs to start at zero (each call writes its own header).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).
 */
int mxgg_grouped_fwd_split_noalloc(const void* a, int64_t lda, const void* a_scales,
                                   int64_t ldas, const void* w, int64_t w_group_stride,
                                   int64_t ldw, const void* w_scales, int64_t ws_group_stride,
                                   int64_t ldws, const int32_t* group_ends, int64_t num_groups,
                                   int64_t M, int64_t N, int64_t K, void* out, int64_t ldo,
                                   int out_dtype, void* stream);

/*
 * Weight-gradient grouped GEMM, contracting over the ragged token dimension:
 *   dw[g] = sum over tokens t of group g of  go_t[:, t] (x) ia_t[:, t]
 * i.e. dW_g = dY_g^T . X_g with both operands stored token-contiguous.
 *   go_t        : e4m3 [N, M], row stride ldgo  (dY transposed)
 *   go_scales_t : E8M0 BLOCK_MAJOR [M/32][ldgos], ldgos >= N   (or NULL)
 *   ia_t        : e4m3 [K, M], row stride ldia  (X transposed)
 *   ia_scales_t : E8M0 BLOCK_MAJOR [M/32][ldias], ldias >= K   (or NULL)
 *                 (strides and bases multiples of 4; readable extent as for
 *                 mxgg_grouped_fwd)
 *   group_ends  : int32 [num_groups] token ends (device).  With scales every
 *                 group bound must be a multiple of 32 (the padded layout that
 *                 mxgg_quant_dim1 produces): a scale block may not span two
 *                 groups, and an expert whose bounds are not multiples of 32 is
 *                 written as NaN.  Without scales the bounds may be any token
 *                 index (ranges off the 16-token load grid are masked token by
 *                 token, at some speed cost for those experts only).
 *   dw          : [num_groups, N, K] bf16 or f32, contiguous, aligned to 4
 *                 elements, K a multiple of 4 (other K: mxgg_grouped_wgrad_strided
 *                 with a row stride rounded up to 4); empty groups are
 *                 written with zeros
 * go_t and ia_t are 16-byte aligned, ldgo and ldia multiples of 16 and at most
 * 2^23, each operand spans less than 2 GiB; strides that are multiples of 128
 * let every load fetch whole cache lines (the fast case).
 *   split_tokens : 0, or split-K: every expert's tokens are cut into chunks
 *                  of split_tokens (a positive multiple of 128) processed as
 *                  separate work items whose partial sums are added to dw
 *                  with fp32 atomics.  Requires out_dtype F32 and dw zeroed
 *                  by the caller; empty experts are then left untouched.  For
 *                  calls with fewer 256x256 output tiles than compute units.
 * Replaces wgrad_fused / wgrad_prepare + wgrad_kernel (wgrad_fused.py:34-112),
 * which restack operands per group and call the forward kernel.
 */
int mxgg_grouped_wgrad(const void* go_t, int64_t ldgo, const void* go_scales_t, int64_t ldgos,
                       const void* ia_t, int64_t ldia, const void* ia_scales_t, int64_t ldias,
                       const int32_t* group_ends, int64_t num_groups,
                       int64_t M, int64_t N, int64_t K,
                       void* dw, int out_dtype, int64_t split_tokens, void* stream);

/*
 * mxgg_grouped_wgrad with split_tokens > 0 and a caller-owned workspace of at
 * least mxgg_grouped_wgrad_workspace_bytes(M, N, K, num_groups, split_tokens)
 * bytes (16-byte aligned, no initialisation): the fp32 partial tiles of
 * experts cut into several chunks go to the workspace and a second kernel on
 * the same stream adds them in chunk order and writes dW (bf16 or fp32).
 * Deterministic, and dW needs no zeroing (experts without tokens are written
 * as zeros).  Same reference interface as mxgg_grouped_wgrad
 * (wgrad_fused.py:22-112); the reference does not split.  Calls that share a
 * workspace must be ordered on one stream.  The size query returns -1 for
 * invalid arguments.
 */
int64_t mxgg_grouped_wgrad_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t num_groups,
                                           int64_t split_tokens);
int mxgg_grouped_wgrad_split(const void* go_t, int64_t ldgo, const void* go_scales_t,
                             int64_t ldgos, const void* ia_t, int64_t ldia,
                             const void* ia_scales_t, int64_t ldias,
                             const int32_t* group_ends, int64_t num_groups,
                             int64_t M, int64_t N, int64_t K,
                             void* dw, int out_dtype, int64_t split_tokens,
                             void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mxgg_grouped_wgrad (workspace == NULL) or mxgg_grouped_wgrad_split
 * (workspace != NULL) writing dW[g][n][k] at element
 * g * ld_dw_expert + n * ld_dw_row + k of dw instead of a contiguous
 * [E, N, K] (ld_dw_row >= K, ld_dw_expert >= (N - 1) * ld_dw_row + K when
 * num_groups > 1, both multiples of 4).  A call over a range of feature rows
 * (rows n0.. of go_t and its scales, or rows k0.. of ia_t and its scales)
 * writes exactly that slice of a larger dW, which is how operands past the
 * 2 GiB buffer range are run: in feature-row chunks, each a whole contraction
 * over every token, so the result equals one launch's.  Replaces the same
 * reference interface, wgrad_fused.py:34-71 (whose per-group restacking,
 * :44-62, has no operand-size limit).
 */
int mxgg_grouped_wgrad_strided(const void* go_t, int64_t ldgo, const void* go_scales_t,
                               int64_t ldgos, const void* ia_t, int64_t ldia,
                               const void* ia_scales_t, int64_t ldias,
                               const int32_t* group_ends, int64_t num_groups,
                               int64_t M, int64_t N, int64_t K,
                               void* dw, int64_t ld_dw_expert, int64_t ld_dw_row,
                               int out_dtype, int64_t split_tokens,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Token routing of a top-k MoE layer on one GPU (the layer's dispatch and
 * combine around the expert GEMMs).  A slot is one (token, k) pair,
 * s = t * topk + k; the routed layout holds one row per slot, grouped by
 * expert, each group padded with empty rows to a multiple of pad_multiple.
 * The reference's trainer gets this layout from torchtitan's token dispatcher,
 * swapped in with pad_multiple = 32 (port_mxfp8.py:214, 240); the dispatcher
 * orders slots by a stable argsort of the expert ids, which is the order here.
 * ------------------------------------------------------------------------- */

/*
 * Dispatch plan, computed on the device by one workgroup (no host sync):
 *   expert_idx  : int32 [tokens, topk] expert of each slot; ids outside
 *                 [0, num_experts) drop the slot
 *   perm        : int32 [tokens * topk] routed row of each slot, -1 if dropped
 *   src         : int32 [rows_cap] slot of each routed row, -1 for padding rows
 *                 and for every row past the last group
 *   group_ends  : int32 [num_experts] cumulative padded group ends (the
 *                 group_ends of the GEMMs and casts over the routed layout)
 *   counts      : int32 [num_experts] slots routed to each expert
 * Slots of one expert keep their slot order.  rows_cap >= tokens * topk +
 * num_experts * (pad_multiple - 1) rows always suffice;
 * 1 <= num_experts <= 1024, 1 <= pad_multiple <= 1024.
 */
int mxgg_route_plan(const int32_t* expert_idx, int64_t tokens, int64_t topk, int64_t num_experts,
                    int64_t pad_multiple, int64_t rows_cap, int32_t* perm, int32_t* src,
                    int32_t* group_ends, int32_t* counts, void* stream);

/*
 * The same plan over many workgroups (one per 4096 slots: a count kernel, one
 * small offsets kernel, a rank kernel), with a caller-owned workspace of at
 * least mxgg_route_plan_workspace_bytes(tokens, topk, num_experts) bytes
 * (4-byte aligned, no initialisation; NULL when that is 0).  Same outputs, bit
 * for bit, as mxgg_route_plan (the stable order is unique); spreading the
 * scattered src stores over many compute units makes it the faster form past
 * a few thousand slots.  Same reference interface as mxgg_route_plan
 * (port_mxfp8.py:214, 240).  Calls that share a workspace must be ordered on
 * one stream.  The size query returns -1 for invalid arguments.
 */
int64_t mxgg_route_plan_workspace_bytes(int64_t tokens, int64_t topk, int64_t num_experts);
int mxgg_route_plan_ws(const int32_t* expert_idx, int64_t tokens, int64_t topk,
                       int64_t num_experts, int64_t pad_multiple, int64_t rows_cap, int32_t* perm,
                       int32_t* src, int32_t* group_ends, int32_t* counts, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * Routed rows in bf16: out[r] = x[src[r] / topk] for src[r] >= 0, times
 * row_scale[src[r]] rounded to bf16 when row_scale (fp32 [tokens * topk]) is
 * given; zero rows for src[r] < 0 and for slots whose token is not below
 * `tokens`.  x: bf16 [tokens, cols] (stride ldx); out: bf16 [rows, cols].
 * cols % 8 == 0, rows 16-byte aligned, strides multiples of 8.  The routed
 * input of the dispatcher (`x[sorted_slots // topk]`), materialised; the MXFP8
 * path uses mxgg_gather_quant_dual instead.
 */
int mxgg_gather_rows(const void* x, int64_t tokens, int64_t cols, int64_t ldx, const int32_t* src,
                     int64_t topk, const float* row_scale, int64_t rows, void* out, int64_t ldo,
                     void* stream);

/*
 * mxgg_quant_dual of the routed rows (as mxgg_gather_rows would write them),
 * read straight from token order: the bf16 routed layout is never written.
 * rows = rows of the routed layout; every other argument as mxgg_quant_dual.
 * Without row_scale: the MXFP8 expert input of the forward pass.  With the
 * combine weights as row_scale and grad_out as x: the MXFP8 casts of the
 * combine's input gradient (the down projection's dY).
 */
int mxgg_gather_quant_dual(const void* x, int64_t tokens, int64_t cols, int64_t ldx,
                           const int32_t* src, int64_t topk, const float* row_scale, int64_t rows,
                           const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap,
                           void* q, int64_t ldq, void* scales, int64_t lds, void* qt, int64_t ldqt,
                           void* scales_t, int64_t ldst, int scale_layout,
                           int32_t* group_ends_pad, int scale_mode, void* stream);

/*
 * mxgg_quant_dim0 of the routed rows (as mxgg_gather_rows would write them
 * without row_scale), read straight from token order: the MXFP8 expert input
 * of a forward-only pass, which needs no token-axis cast.  rows = rows of the
 * routed layout (every row is written; padding rows as zero blocks); every
 * other argument as mxgg_quant_dim0.  cols <= 65535 * 512 (else
 * MXGG_ERR_UNSUPPORTED).
 */
int mxgg_gather_quant_dim0(const void* x, int64_t tokens, int64_t cols, int64_t ldx,
                           const int32_t* src, int64_t topk, int64_t rows, void* q, int64_t ldq,
                           void* scales, int64_t lds, int scale_layout, int scale_mode,
                           void* stream);

/*
 * Combine: out[t] = bf16(sum over k of float(bf16(float(y[perm[s]]) *
 * scores[s]))), s = t * topk + k, summed in fp32 in k order (one rounding of
 * the sum); without scores each term is the row itself.  Slots with perm < 0
 * or perm >= rows add nothing.  y: bf16 [rows, cols] routed layout; out: bf16
 * [tokens, cols].  cols % 8 == 0, 16-byte aligned rows.  The dispatcher's
 * weighted scatter-add back to token order; without scores, the input
 * gradient of the gather (dX from the routed dX).
 */
int mxgg_combine(const void* y, int64_t rows, int64_t cols, int64_t ldy, const int32_t* perm,
                 const float* scores, int64_t tokens, int64_t topk, void* out, int64_t ldo,
                 void* stream);

/*
 * Gradient of the combine with respect to its weights:
 *   grad_scores[s] = sum over h of float(grad_out[t][h]) * float(y[perm[s]][h])
 * (fp32), 0 for a dropped slot.  grad_out: bf16 [tokens, cols]; y as in
 * mxgg_combine; grad_scores: fp32 [tokens * topk].
 */
int mxgg_combine_score_grad(const void* grad_out, int64_t ldg, const void* y, int64_t rows,
                            int64_t cols, int64_t ldy, const int32_t* perm, int64_t tokens,
                            int64_t topk, float* grad_scores, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXGG_H */
