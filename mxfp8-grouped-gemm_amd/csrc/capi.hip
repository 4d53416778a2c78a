// extern "C" entry points of libmxgg.so: argument validation, then launch.
// No entry point allocates, frees or synchronises; all launches go to the
// caller's stream.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "mxgg_internal.h"

namespace mxgg {

namespace {
thread_local char g_last_error[512] = "";

constexpr int64_t kMaxGroupsAbi = 1024;
constexpr int64_t kMaxBufferBytes = 0x7FFFFFF0LL;  // one buffer resource per operand
// GEMM tiles run up to 255 rows past an operand's last row; those offsets must
// stay below 2^32 (they read as zero through the buffer range check).
constexpr int64_t kMaxRowStride = INT64_C(1) << 23;
// Kernels with one wave per row and four rows per 256-thread workgroup: the
// grid holds at most 2^32 - 1 work-items.
constexpr int64_t kMaxWaveRows = 4 * ((INT64_C(1) << 24) - 1);

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return -1;
    cache[dev] = n;
  }
  return cache[dev];
}

static int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return set_error(MXGG_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MXGG_OK;
}

}  // namespace mxgg

using namespace mxgg;

extern "C" {

int mxgg_abi_version(void) { return MXGG_ABI_VERSION; }

const char* mxgg_status_string(int status) {
  switch (status) {
    case MXGG_OK: return "ok";
    case MXGG_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MXGG_ERR_SHAPE: return "bad shape";
    case MXGG_ERR_ALIGNMENT: return "misaligned pointer or leading dimension";
    case MXGG_ERR_UNSUPPORTED: return "unsupported size";
    case MXGG_ERR_DEVICE: return "device error";
    case MXGG_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

const char* mxgg_last_error(void) { return g_last_error; }

static bool valid_layout(int layout) {
  return layout == MXGG_SCALES_ROW_MAJOR || layout == MXGG_SCALES_BLOCK_MAJOR;
}

static int check_dim0(const char* what, const void* x, int64_t rows, int64_t cols, int64_t ldx,
                      const void* q, int64_t ldq, const void* scales, int64_t lds,
                      int scale_layout, int scale_mode) {
  const int mode = scale_mode & 0xFF;
  if (mode != MXGG_SCALE_RCEIL && mode != MXGG_SCALE_FLOOR)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: unknown scale_mode %d", what, scale_mode);
  if (!valid_layout(scale_layout))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: unknown scale_layout %d", what,
                     scale_layout);
  if (rows < 0 || cols < 0)
    return set_error(MXGG_ERR_SHAPE, "%s: negative size rows=%lld cols=%lld", what,
                     (long long)rows, (long long)cols);
  if (cols % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "%s: cols=%lld is not a multiple of 32", what,
                     (long long)cols);
  if (cols > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "%s: cols above 2^31", what);
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!x || !q || !scales) return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: null pointer", what);
  if (ldx < cols || ldq < cols ||
      lds < (scale_layout == MXGG_SCALES_BLOCK_MAJOR ? rows : cols / 32))
    return set_error(MXGG_ERR_SHAPE, "%s: leading dimension smaller than the row", what);
  if (!aligned16(x) || !aligned16(q) || ldx % 8 != 0 || ldq % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(q) & 7u) != 0)
    return set_error(MXGG_ERR_ALIGNMENT,
                     "%s: x and q must be 16-byte aligned, ldx and ldq multiples of 8", what);
  return MXGG_OK;
}

int mxgg_quant_dim0(const void* x, int64_t rows, int64_t cols, int64_t ldx, void* q, int64_t ldq,
                    void* scales, int64_t lds, int scale_layout, int scale_mode, void* stream) {
  const int st = check_dim0("quant_dim0", x, rows, cols, ldx, q, ldq, scales, lds, scale_layout,
                            scale_mode);
  if (st != MXGG_OK || rows == 0 || cols == 0) return st;
  return check_launch(launch_quant_dim0(static_cast<const uint16_t*>(x), rows, cols, ldx,
                                        static_cast<uint8_t*>(q), ldq,
                                        static_cast<uint8_t*>(scales), lds, scale_layout,
                                        scale_mode, static_cast<hipStream_t>(stream)),
                      "quant_dim0");
}

int mxgg_quant_dim1(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                    const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap,
                    void* qt, int64_t ldqt, void* scales_t, int64_t ldst, int scale_layout,
                    int32_t* group_ends_pad, int scale_mode, void* stream) {
  const int mode = scale_mode & 0xFF;
  if (mode != MXGG_SCALE_RCEIL && mode != MXGG_SCALE_FLOOR)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "quant_dim1: unknown scale_mode %d", scale_mode);
  if (!valid_layout(scale_layout))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "quant_dim1: unknown scale_layout %d",
                     scale_layout);
  if (rows < 0 || cols < 0 || rows_pad_cap < 0)
    return set_error(MXGG_ERR_SHAPE, "quant_dim1: negative size");
  if (cols % 8 != 0)
    return set_error(MXGG_ERR_SHAPE, "quant_dim1: cols=%lld is not a multiple of 8",
                     (long long)cols);
  if (rows_pad_cap % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "quant_dim1: rows_pad_cap=%lld is not a multiple of 32",
                     (long long)rows_pad_cap);
  if (group_ends) {
    if (num_groups < 1 || num_groups > kMaxGroupsAbi)
      return set_error(MXGG_ERR_UNSUPPORTED, "quant_dim1: num_groups=%lld outside [1, %lld]",
                       (long long)num_groups, (long long)kMaxGroupsAbi);
    if (!group_ends_pad)
      return set_error(MXGG_ERR_INVALID_ARGUMENT,
                       "quant_dim1: group_ends_pad is required with group_ends");
  }
  const int64_t groups = group_ends ? num_groups : 1;
  const int64_t need = ((rows + 31 * (group_ends ? groups : 0) + 31) / 32) * 32;
  if (rows_pad_cap < need)
    return set_error(MXGG_ERR_SHAPE, "quant_dim1: rows_pad_cap=%lld < required %lld",
                     (long long)rows_pad_cap, (long long)need);
  if (cols == 0 || rows_pad_cap == 0) return MXGG_OK;
  if (!x && rows > 0) return set_error(MXGG_ERR_INVALID_ARGUMENT, "quant_dim1: null x");
  if (!qt || !scales_t) return set_error(MXGG_ERR_INVALID_ARGUMENT, "quant_dim1: null output");
  if (ldx < cols || ldqt < rows_pad_cap ||
      ldst < (scale_layout == MXGG_SCALES_BLOCK_MAJOR ? cols : rows_pad_cap / 32))
    return set_error(MXGG_ERR_SHAPE, "quant_dim1: leading dimension smaller than the row");
  if ((x && !aligned16(x)) || !aligned16(qt) || ldx % 8 != 0 || ldqt % 16 != 0)
    return set_error(MXGG_ERR_ALIGNMENT,
                     "quant_dim1: x and qt must be 16-byte aligned, ldx % 8 == 0, ldqt % 16 == 0");
  if (rows > INT32_MAX || rows_pad_cap > INT32_MAX || cols > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "quant_dim1: more than 2^31 rows or columns");
  return check_launch(
      launch_quant_dim1(static_cast<const uint16_t*>(x), rows, cols, ldx, group_ends, groups,
                        rows_pad_cap, static_cast<uint8_t*>(qt), ldqt,
                        static_cast<uint8_t*>(scales_t), ldst, scale_layout, group_ends_pad,
                        scale_mode, static_cast<hipStream_t>(stream)),
      "quant_dim1");
}

// Argument rules shared by the dual casts (plain and gathered); returns
// MXGG_OK, or the status with the error message set, naming `what`.
static int check_dual(const char* what, bool have_x, int64_t rows, int64_t cols, int64_t ldx,
                      const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap,
                      const void* q, int64_t ldq, const void* scales, int64_t lds, const void* qt,
                      int64_t ldqt, const void* scales_t, int64_t ldst, int scale_layout,
                      const int32_t* group_ends_pad, int scale_mode, const void* x) {
  const int mode = scale_mode & 0xFF;
  if (mode != MXGG_SCALE_RCEIL && mode != MXGG_SCALE_FLOOR)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: unknown scale_mode %d", what, scale_mode);
  if (!valid_layout(scale_layout))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: unknown scale_layout %d", what,
                     scale_layout);
  if (rows < 0 || cols < 0 || rows_pad_cap < 0)
    return set_error(MXGG_ERR_SHAPE, "%s: negative size", what);
  if (cols % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "%s: cols=%lld is not a multiple of 32", what,
                     (long long)cols);
  if (rows_pad_cap % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "%s: rows_pad_cap=%lld is not a multiple of 32", what,
                     (long long)rows_pad_cap);
  if (group_ends) {
    if (num_groups < 1 || num_groups > kMaxGroupsAbi)
      return set_error(MXGG_ERR_UNSUPPORTED, "%s: num_groups=%lld outside [1, %lld]", what,
                       (long long)num_groups, (long long)kMaxGroupsAbi);
    if (!group_ends_pad)
      return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: group_ends_pad is required with group_ends",
                       what);
  }
  const int64_t need = ((rows + 31 * (group_ends ? num_groups : 0) + 31) / 32) * 32;
  if (rows_pad_cap < need)
    return set_error(MXGG_ERR_SHAPE, "%s: rows_pad_cap=%lld < required %lld", what,
                     (long long)rows_pad_cap, (long long)need);
  if (cols == 0 || rows_pad_cap == 0) return MXGG_OK;
  if (rows > 0 && (!have_x || !q || !scales))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: null x, q or scales", what);
  if (!qt || !scales_t) return set_error(MXGG_ERR_INVALID_ARGUMENT, "%s: null qt", what);
  const bool bm = scale_layout == MXGG_SCALES_BLOCK_MAJOR;
  if (ldx < cols || ldq < cols || lds < (bm ? rows : cols / 32) || ldqt < rows_pad_cap ||
      ldst < (bm ? cols : rows_pad_cap / 32))
    return set_error(MXGG_ERR_SHAPE, "%s: leading dimension smaller than the row", what);
  if ((x && !aligned16(x)) || ldx % 8 != 0 || (q && (reinterpret_cast<uintptr_t>(q) & 7u) != 0) ||
      ldq % 8 != 0 || !aligned16(qt) || ldqt % 16 != 0)
    return set_error(MXGG_ERR_ALIGNMENT,
                     "%s: x 16-byte aligned with ldx %% 8 == 0, q 8-byte aligned with ldq "
                     "%% 8 == 0, qt 16-byte aligned with ldqt %% 16 == 0",
                     what);
  if (rows > INT32_MAX || rows_pad_cap > INT32_MAX || cols > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "%s: more than 2^31 rows or columns", what);
  return MXGG_OK;
}

int mxgg_quant_dual(const void* x, int64_t rows, int64_t cols, int64_t ldx,
                    const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap, void* q,
                    int64_t ldq, void* scales, int64_t lds, void* qt, int64_t ldqt,
                    void* scales_t, int64_t ldst, int scale_layout, int32_t* group_ends_pad,
                    int scale_mode, void* stream) {
  const int st = check_dual("quant_dual", x != nullptr, rows, cols, ldx, group_ends, num_groups,
                            rows_pad_cap, q, ldq, scales, lds, qt, ldqt, scales_t, ldst,
                            scale_layout, group_ends_pad, scale_mode, x);
  if (st != MXGG_OK || cols == 0 || rows_pad_cap == 0) return st;
  return check_launch(
      launch_quant_dual(static_cast<const uint16_t*>(x), rows, cols, ldx, group_ends,
                        group_ends ? num_groups : 1, rows_pad_cap, static_cast<uint8_t*>(q), ldq,
                        static_cast<uint8_t*>(scales), lds, static_cast<uint8_t*>(qt), ldqt,
                        static_cast<uint8_t*>(scales_t), ldst, scale_layout, group_ends_pad,
                        scale_mode, static_cast<hipStream_t>(stream)),
      "quant_dual");
}

int mxgg_swiglu_quant_dim0(const void* gate, const void* up, int64_t ldh, int64_t rows,
                           int64_t cols, void* a_out, int64_t lda, void* q, int64_t ldq,
                           void* scales, int64_t lds, int scale_layout, int scale_mode,
                           void* stream) {
  const int mode = scale_mode & 0xFF;
  if (mode != MXGG_SCALE_RCEIL && mode != MXGG_SCALE_FLOOR)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_quant_dim0: unknown scale_mode %d",
                     scale_mode);
  if (!valid_layout(scale_layout))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_quant_dim0: unknown scale_layout %d",
                     scale_layout);
  if (rows < 0 || cols < 0)
    return set_error(MXGG_ERR_SHAPE, "swiglu_quant_dim0: negative size");
  if (cols % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "swiglu_quant_dim0: cols=%lld is not a multiple of 32",
                     (long long)cols);
  if (cols > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "swiglu_quant_dim0: cols above 2^31");
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!gate || !up || !q || !scales)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_quant_dim0: null pointer");
  if (ldh < cols || ldq < cols || (a_out && lda < cols) ||
      lds < (scale_layout == MXGG_SCALES_BLOCK_MAJOR ? rows : cols / 32))
    return set_error(MXGG_ERR_SHAPE, "swiglu_quant_dim0: leading dimension smaller than the row");
  if (!aligned16(gate) || !aligned16(up) || ldh % 8 != 0 || ldq % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(q) & 7u) != 0 || (a_out && (!aligned16(a_out) || lda % 8 != 0)))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "swiglu_quant_dim0: gate, up and a_out 16-byte aligned with strides multiples "
                     "of 8; q 8-byte aligned with ldq %% 8 == 0");
  return check_launch(
      launch_swiglu_quant_dim0(static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                               ldh, rows, cols, static_cast<uint16_t*>(a_out), lda,
                               static_cast<uint8_t*>(q), ldq, static_cast<uint8_t*>(scales), lds,
                               scale_layout, scale_mode, static_cast<hipStream_t>(stream)),
      "swiglu_quant_dim0");
}

int mxgg_swiglu_bwd_quant(const void* gate, const void* up, int64_t ldh, const void* grad_a,
                          int64_t ldga, int64_t rows, int64_t cols, const int32_t* group_ends,
                          int64_t num_groups, int64_t rows_pad_cap, void* dh_q, int64_t lddq,
                          void* dh_scales, int64_t ldds, void* dh_qt, int64_t lddqt,
                          void* dh_scales_t, int64_t lddst, void* a_qt, int64_t ldaqt,
                          void* a_scales_t, int64_t ldast, int32_t* group_ends_pad, void* dh_out,
                          int64_t lddh, int scale_layout, int scale_mode, void* stream) {
  const int mode = scale_mode & 0xFF;
  if (mode != MXGG_SCALE_RCEIL && mode != MXGG_SCALE_FLOOR)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_bwd_quant: unknown scale_mode %d",
                     scale_mode);
  if (!valid_layout(scale_layout))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_bwd_quant: unknown scale_layout %d",
                     scale_layout);
  if (rows < 0 || cols < 0 || rows_pad_cap < 0)
    return set_error(MXGG_ERR_SHAPE, "swiglu_bwd_quant: negative size");
  if (cols % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "swiglu_bwd_quant: cols=%lld is not a multiple of 32",
                     (long long)cols);
  if (rows_pad_cap % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "swiglu_bwd_quant: rows_pad_cap=%lld not a multiple of 32",
                     (long long)rows_pad_cap);
  if (group_ends) {
    if (num_groups < 1 || num_groups > kMaxGroupsAbi)
      return set_error(MXGG_ERR_UNSUPPORTED,
                       "swiglu_bwd_quant: num_groups=%lld outside [1, %lld]",
                       (long long)num_groups, (long long)kMaxGroupsAbi);
    if (!group_ends_pad)
      return set_error(MXGG_ERR_INVALID_ARGUMENT,
                       "swiglu_bwd_quant: group_ends_pad is required with group_ends");
  }
  const int64_t need = ((rows + 31 * (group_ends ? num_groups : 0) + 31) / 32) * 32;
  if (rows_pad_cap < need)
    return set_error(MXGG_ERR_SHAPE, "swiglu_bwd_quant: rows_pad_cap=%lld < required %lld",
                     (long long)rows_pad_cap, (long long)need);
  if (cols == 0 || rows_pad_cap == 0) return MXGG_OK;
  if (rows > 0 && (!gate || !up || !grad_a || !dh_q || !dh_scales))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_bwd_quant: null input or dh_q");
  if (!dh_qt || !dh_scales_t || !a_qt || !a_scales_t)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "swiglu_bwd_quant: null token-axis output");
  const bool bm = scale_layout == MXGG_SCALES_BLOCK_MAJOR;
  if (ldh < cols || ldga < cols || lddq < 2 * cols || (dh_out && lddh < 2 * cols) ||
      ldds < (bm ? rows : 2 * cols / 32) || lddqt < rows_pad_cap || ldaqt < rows_pad_cap ||
      lddst < (bm ? 2 * cols : rows_pad_cap / 32) || ldast < (bm ? cols : rows_pad_cap / 32))
    return set_error(MXGG_ERR_SHAPE, "swiglu_bwd_quant: leading dimension smaller than the row");
  const uintptr_t in_bits = reinterpret_cast<uintptr_t>(gate) |
                            reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(grad_a);
  if ((in_bits & 15u) != 0 || ldh % 8 != 0 || ldga % 8 != 0 ||
      (dh_out && (!aligned16(dh_out) || lddh % 8 != 0)))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "swiglu_bwd_quant: gate, up, grad_a and dh_out 16-byte aligned with strides "
                     "multiples of 8");
  if ((reinterpret_cast<uintptr_t>(dh_q) & 7u) != 0 || lddq % 8 != 0 || !aligned16(dh_qt) ||
      !aligned16(a_qt) || lddqt % 16 != 0 || ldaqt % 16 != 0)
    return set_error(MXGG_ERR_ALIGNMENT,
                     "swiglu_bwd_quant: dh_q 8-byte aligned with lddq %% 8 == 0; dh_qt and a_qt "
                     "16-byte aligned with strides multiples of 16");
  // one-dimensional grid of 256-thread workgroups: at most 2^24 - 1 of them
  const int64_t wgs = ((rows_pad_cap + 127) / 128) * ((cols + 127) / 128);
  if (rows > INT32_MAX || rows_pad_cap > INT32_MAX || cols > INT32_MAX || wgs >= (INT64_C(1) << 24))
    return set_error(MXGG_ERR_UNSUPPORTED,
                     "swiglu_bwd_quant: rows or rows_pad_cap above 2^31, or "
                     "ceil(rows_pad_cap/128) * ceil(cols/128) = %lld workgroups (at most 2^24 - 1)",
                     (long long)wgs);
  SwigluBwdLaunch l;
  l.gate = static_cast<const uint16_t*>(gate);
  l.up = static_cast<const uint16_t*>(up);
  l.da = static_cast<const uint16_t*>(grad_a);
  l.group_ends = group_ends;
  l.group_ends_pad = group_ends_pad;
  l.dq = static_cast<uint8_t*>(dh_q);
  l.ds = static_cast<uint8_t*>(dh_scales);
  l.dqt = static_cast<uint8_t*>(dh_qt);
  l.dst = static_cast<uint8_t*>(dh_scales_t);
  l.aqt = static_cast<uint8_t*>(a_qt);
  l.ast = static_cast<uint8_t*>(a_scales_t);
  l.dh = static_cast<uint16_t*>(dh_out);
  l.ldh = ldh;
  l.ldda = ldga;
  l.rows = rows;
  l.cols = cols;
  l.num_groups = group_ends ? num_groups : 1;
  l.cap = rows_pad_cap;
  l.lddq = lddq;
  l.ldds = ldds;
  l.lddqt = lddqt;
  l.lddst = lddst;
  l.ldaqt = ldaqt;
  l.ldast = ldast;
  l.lddh = lddh;
  l.layout = scale_layout;
  l.mode = scale_mode;
  return check_launch(launch_swiglu_bwd_quant(l, static_cast<hipStream_t>(stream)),
                      "swiglu_bwd_quant");
}

int mxgg_scales_to_block_major(const void* src, int64_t batch, int64_t rows, int64_t nblk,
                               int64_t src_bstride, int64_t lds, void* dst,
                               int64_t dst_bstride, int64_t ldd, void* stream) {
  if (batch < 0 || rows < 0 || nblk < 0)
    return set_error(MXGG_ERR_SHAPE, "scales_to_block_major: negative size");
  if (batch == 0 || rows == 0 || nblk == 0) return MXGG_OK;
  if (!src || !dst)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "scales_to_block_major: null pointer");
  if (lds < nblk || ldd < rows || (batch > 1 && (src_bstride < rows * lds ||
                                                  dst_bstride < nblk * ldd)))
    return set_error(MXGG_ERR_SHAPE, "scales_to_block_major: strides smaller than the data");
  if (batch > 65535)
    return set_error(MXGG_ERR_UNSUPPORTED, "scales_to_block_major: batch above 65535");
  return check_launch(
      launch_scales_to_block_major(static_cast<const uint8_t*>(src), batch, rows, nblk,
                                   src_bstride, lds, static_cast<uint8_t*>(dst), dst_bstride,
                                   ldd, static_cast<hipStream_t>(stream)),
      "scales_to_block_major");
}

int mxgg_offs_to_group_ends(const int32_t* offs, int64_t num_groups, int64_t tokens,
                            int offs_kind, int32_t* group_ends, void* stream) {
  if (offs_kind != MXGG_OFFS_ENDS && offs_kind != MXGG_OFFS_SIZES && offs_kind != MXGG_OFFS_AUTO)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "offs_to_group_ends: unknown offs_kind %d",
                     offs_kind);
  if (num_groups < 1 || num_groups > kMaxGroupsAbi)
    return set_error(MXGG_ERR_UNSUPPORTED, "offs_to_group_ends: num_groups=%lld outside [1, %lld]",
                     (long long)num_groups, (long long)kMaxGroupsAbi);
  if (tokens < 0) return set_error(MXGG_ERR_SHAPE, "offs_to_group_ends: negative tokens");
  if (!offs || !group_ends)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "offs_to_group_ends: null pointer");
  if (offs == group_ends)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "offs_to_group_ends: group_ends aliases offs");
  return check_launch(launch_offs_to_ends(offs, num_groups, tokens, offs_kind, group_ends,
                                          static_cast<hipStream_t>(stream)),
                      "offs_to_group_ends");
}

int mxgg_zero_rows_past_groups(void* out, int64_t rows, int64_t row_bytes, int64_t ld_bytes,
                               const int32_t* group_ends, int64_t num_groups, void* stream) {
  if (rows < 0 || row_bytes < 0 || ld_bytes < row_bytes)
    return set_error(MXGG_ERR_SHAPE, "zero_rows_past_groups: rows=%lld row_bytes=%lld ld=%lld",
                     (long long)rows, (long long)row_bytes, (long long)ld_bytes);
  if (num_groups < 1 || num_groups > kMaxGroupsAbi)
    return set_error(MXGG_ERR_UNSUPPORTED,
                     "zero_rows_past_groups: num_groups=%lld outside [1, %lld]",
                     (long long)num_groups, (long long)kMaxGroupsAbi);
  if (rows == 0 || row_bytes == 0) return MXGG_OK;
  if (!out || !group_ends)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "zero_rows_past_groups: null pointer");
  if (!aligned16(out) || row_bytes % 16 != 0 || ld_bytes % 16 != 0)
    return set_error(MXGG_ERR_ALIGNMENT,
                     "zero_rows_past_groups: out, row_bytes and ld_bytes must be multiples of 16");
  if (rows > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "zero_rows_past_groups: rows above 2^31");
  return check_launch(launch_zero_tail(static_cast<uint8_t*>(out), rows, row_bytes, ld_bytes,
                                       group_ends, num_groups, static_cast<hipStream_t>(stream)),
                      "zero_rows_past_groups");
}

// Outputs of the fused SwiGLU forward (mxgg_grouped_fwd_swiglu_quant).
struct SwigluOut {
  void* q;
  int64_t ldq;
  void* scales;
  int64_t lds;
  int layout, mode;
};

static int grouped_fwd(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                       const void* w, int64_t w_group_stride, int64_t ldw, const void* w_scales,
                       int64_t ws_group_stride, int64_t ldws, const int32_t* group_ends,
                       int64_t num_groups, int64_t M, int64_t N, int64_t K, void* out,
                       int64_t ldo, int out_dtype, void* workspace, void* stream,
                       const SwigluOut* sw = nullptr) {
  if (!sw && out_dtype != MXGG_OUT_BF16 && out_dtype != MXGG_OUT_F32)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_fwd: unknown out_dtype %d", out_dtype);
  if (M < 0 || N < 0 || K < 0)
    return set_error(MXGG_ERR_SHAPE, "grouped_fwd: negative size");
  if (K % 32 != 0 || K == 0)
    return set_error(MXGG_ERR_SHAPE, "grouped_fwd: K=%lld must be a positive multiple of 32",
                     (long long)K);
  const bool scaled = a_scales != nullptr;
  if ((a_scales == nullptr) != (w_scales == nullptr))
    return set_error(MXGG_ERR_INVALID_ARGUMENT,
                     "grouped_fwd: a_scales and w_scales must both be given or both be NULL");
  const int64_t E = group_ends ? num_groups : 1;
  if (E < 1 || E > kMaxGroupsAbi)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_fwd: num_groups=%lld outside [1, %lld]",
                     (long long)num_groups, (long long)kMaxGroupsAbi);
  if (M == 0 || N == 0) return MXGG_OK;
  if (!a || !w || (!sw && !out))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_fwd: null pointer");
  if (lda < K || ldw < K || (!sw && ldo < N) || (scaled && (ldas < M || ldws < N)))
    return set_error(MXGG_ERR_SHAPE,
                     "grouped_fwd: leading dimension smaller than the row (block-major scales: "
                     "ldas >= M, ldws >= N)");
  // Experts may overlap or interleave (they are only read): the transposed
  // weights of dgrad hold expert e in columns [e*N, (e+1)*N) of one matrix.
  if (E > 1 && (w_group_stride < 0 || (scaled && ws_group_stride < 0)))
    return set_error(MXGG_ERR_SHAPE, "grouped_fwd: negative expert stride");
  if (scaled && ((reinterpret_cast<uintptr_t>(a_scales) | reinterpret_cast<uintptr_t>(w_scales)) %
                     4 != 0 ||
                 ldas % 4 != 0 || ldws % 4 != 0 || (E > 1 && ws_group_stride % 4 != 0)))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "grouped_fwd: scale bases, strides and expert stride must be multiples of 4");
  if (scaled && ((K / 32) * ldas > kMaxBufferBytes || (K / 32) * ldws > kMaxBufferBytes ||
                 (E - 1) * ws_group_stride + (K / 32) * ldws > INT64_C(1) << 40))
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_fwd: scale array larger than 2 GiB");
  if (!aligned16(a) || !aligned16(w) || lda % 16 != 0 || ldw % 16 != 0 ||
      (E > 1 && w_group_stride % 16 != 0))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "grouped_fwd: a and w must be 16-byte aligned with lda, ldw and the expert "
                     "stride multiples of 16");
  const int esz = out_dtype == MXGG_OUT_F32 ? 4 : 2;
  if (!sw && ((reinterpret_cast<uintptr_t>(out) % (4 * esz)) != 0 || ldo % 4 != 0))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "grouped_fwd: out must be aligned to 4 elements with ldo % 4 == 0");
  if ((M - 1) * lda + K > kMaxBufferBytes || (N - 1) * ldw + K > kMaxBufferBytes)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_fwd: operand larger than 2 GiB");
  if (lda > kMaxRowStride || ldw > kMaxRowStride)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_fwd: row stride above 8 MiB");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_fwd: dimension above 2^31");
  FwdArgs args;
  args.a = static_cast<const uint8_t*>(a);
  args.as = static_cast<const uint8_t*>(a_scales);
  args.w = static_cast<const uint8_t*>(w);
  args.ws = static_cast<const uint8_t*>(w_scales);
  args.group_ends = group_ends;
  args.out = out;
  args.lda = lda;
  args.ldas = scaled ? ldas : 0;
  args.w_gstride = w_group_stride;
  args.ldw = ldw;
  args.ws_gstride = scaled ? ws_group_stride : 0;
  args.ldws = scaled ? ldws : 0;
  args.ldo = ldo;
  args.M = (int32_t)M;
  args.N = (int32_t)N;
  args.K = (int32_t)K;
  args.E = (int32_t)E;
  args.out_f32 = out_dtype == MXGG_OUT_F32;
  args.scaled = scaled;
  args.split_ws = static_cast<float*>(workspace);
  args.swiglu_mode = -1;
  args.aq = nullptr;
  args.as_out = nullptr;
  args.ldaq = args.as_row = args.as_blk = 0;
  if (sw) {
    const bool bm = sw->layout == MXGG_SCALES_BLOCK_MAJOR;
    args.swiglu_mode = sw->mode;
    args.aq = static_cast<uint8_t*>(sw->q);
    args.as_out = static_cast<uint8_t*>(sw->scales);
    args.ldaq = sw->ldq;
    args.as_row = bm ? 1 : sw->lds;
    args.as_blk = bm ? sw->lds : 1;
  }
  return check_launch(launch_grouped_fwd(args, static_cast<hipStream_t>(stream)), "grouped_fwd");
}

int mxgg_grouped_fwd(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                     const void* w, int64_t w_group_stride, int64_t ldw, const void* w_scales,
                     int64_t ws_group_stride, int64_t ldws, const int32_t* group_ends,
                     int64_t num_groups, int64_t M, int64_t N, int64_t K, void* out, int64_t ldo,
                     int out_dtype, void* stream) {
  return grouped_fwd(a, lda, a_scales, ldas, w, w_group_stride, ldw, w_scales, ws_group_stride,
                     ldws, group_ends, num_groups, M, N, K, out, ldo, out_dtype, nullptr, stream);
}

int64_t mxgg_grouped_fwd_workspace_bytes(void) { return fwd_split_workspace_bytes(); }

static int grouped_fwd_swiglu(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                              const void* w, int64_t w_group_stride, int64_t ldw,
                              const void* w_scales, int64_t ws_group_stride, int64_t ldws,
                              const int32_t* group_ends, int64_t num_groups, int64_t M, int64_t F,
                              int64_t K, void* h, int64_t ldh, void* q, int64_t ldq, void* scales,
                              int64_t lds, int scale_layout, int scale_mode, void* stream) {
  if (scale_mode != MXGG_SCALE_RCEIL && scale_mode != MXGG_SCALE_FLOOR)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_fwd_swiglu_quant: unknown scale_mode %d",
                     scale_mode);
  if (!valid_layout(scale_layout))
    return set_error(MXGG_ERR_INVALID_ARGUMENT,
                     "grouped_fwd_swiglu_quant: unknown scale_layout %d", scale_layout);
  if (F < 0 || F % 128 != 0)
    return set_error(MXGG_ERR_SHAPE,
                     "grouped_fwd_swiglu_quant: F=%lld must be a non-negative multiple of 128",
                     (long long)F);
  if (F > (INT64_C(1) << 29))
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_fwd_swiglu_quant: F above 2^29");
  if (M > 0 && F > 0) {
    if (!q || !scales)
      return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_fwd_swiglu_quant: null output");
    const bool bm = scale_layout == MXGG_SCALES_BLOCK_MAJOR;
    if (ldq < F || lds < (bm ? M : F / 32))
      return set_error(MXGG_ERR_SHAPE,
                       "grouped_fwd_swiglu_quant: leading dimension smaller than the row");
    if ((reinterpret_cast<uintptr_t>(q) & 7u) != 0 || ldq % 8 != 0)
      return set_error(MXGG_ERR_ALIGNMENT,
                       "grouped_fwd_swiglu_quant: q must be 8-byte aligned with ldq %% 8 == 0");
    if (h && ldh < 2 * F)
      return set_error(MXGG_ERR_SHAPE, "grouped_fwd_swiglu_quant: ldh smaller than 2F");
    if (h && (!aligned16(h) || ldh % 8 != 0))
      return set_error(MXGG_ERR_ALIGNMENT,
                       "grouped_fwd_swiglu_quant: h must be 16-byte aligned with ldh %% 8 == 0");
  }
  const SwigluOut sw{q, ldq, scales, lds, scale_layout, scale_mode};
  return grouped_fwd(a, lda, a_scales, ldas, w, w_group_stride, ldw, w_scales, ws_group_stride,
                     ldws, group_ends, num_groups, M, 2 * F, K, h, h ? ldh : 0, MXGG_OUT_BF16,
                     nullptr, stream, &sw);
}

int mxgg_grouped_fwd_swiglu_quant(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                                  const void* w, int64_t w_group_stride, int64_t ldw,
                                  const void* w_scales, int64_t ws_group_stride, int64_t ldws,
                                  const int32_t* group_ends, int64_t num_groups, int64_t M,
                                  int64_t F, int64_t K, void* q, int64_t ldq, void* scales,
                                  int64_t lds, int scale_layout, int scale_mode, void* stream) {
  return grouped_fwd_swiglu(a, lda, a_scales, ldas, w, w_group_stride, ldw, w_scales,
                            ws_group_stride, ldws, group_ends, num_groups, M, F, K, nullptr, 0, q,
                            ldq, scales, lds, scale_layout, scale_mode, stream);
}

int mxgg_grouped_fwd_swiglu_quant_keep_h(const void* a, int64_t lda, const void* a_scales,
                                         int64_t ldas, const void* w, int64_t w_group_stride,
                                         int64_t ldw, const void* w_scales,
                                         int64_t ws_group_stride, int64_t ldws,
                                         const int32_t* group_ends, int64_t num_groups, int64_t M,
                                         int64_t F, int64_t K, void* h, int64_t ldh, void* q,
                                         int64_t ldq, void* scales, int64_t lds, int scale_layout,
                                         int scale_mode, void* stream) {
  if (M > 0 && F > 0 && !h)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_fwd_swiglu_quant: null h");
  return grouped_fwd_swiglu(a, lda, a_scales, ldas, w, w_group_stride, ldw, w_scales,
                            ws_group_stride, ldws, group_ends, num_groups, M, F, K, h, ldh, q, ldq,
                            scales, lds, scale_layout, scale_mode, stream);
}

int mxgg_grouped_fwd_split(const void* a, int64_t lda, const void* a_scales, int64_t ldas,
                           const void* w, int64_t w_group_stride, int64_t ldw,
                           const void* w_scales, int64_t ws_group_stride, int64_t ldws,
                           const int32_t* group_ends, int64_t num_groups, int64_t M, int64_t N,
                           int64_t K, void* out, int64_t ldo, int out_dtype, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  if (!workspace)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_fwd_split: null workspace");
  if (workspace_bytes < fwd_split_workspace_bytes())
    return set_error(MXGG_ERR_SHAPE, "grouped_fwd_split: workspace_bytes=%lld < %lld",
                     (long long)workspace_bytes, (long long)fwd_split_workspace_bytes());
  if (!aligned16(workspace))
    return set_error(MXGG_ERR_ALIGNMENT, "grouped_fwd_split: workspace must be 16-byte aligned");
  return grouped_fwd(a, lda, a_scales, ldas, w, w_group_stride, ldw, w_scales, ws_group_stride,
                     ldws, group_ends, num_groups, M, N, K, out, ldo, out_dtype, workspace,
                     stream);
}

int mxgg_grouped_fwd_split_noalloc(const void* a, int64_t lda, const void* a_scales,
                                   int64_t ldas, const void* w, int64_t w_group_stride,
                                   int64_t ldw, const void* w_scales, int64_t ws_group_stride,
                                   int64_t ldws, const int32_t* group_ends, int64_t num_groups,
                                   int64_t M, int64_t N, int64_t K, void* out, int64_t ldo,
                                   int out_dtype, void* stream) {
  const int64_t need = fwd_split_workspace_bytes();
  if (need > noalloc_scratch_bytes())
    return set_error(MXGG_ERR_UNSUPPORTED,
                     "grouped_fwd_split_noalloc: this device needs %lld bytes of split scratch, "
                     "the library holds %lld (at most 256 compute units)",
                     (long long)need, (long long)noalloc_scratch_bytes());
  void* ws = noalloc_scratch();
  if (ws == nullptr)
    return set_error(MXGG_ERR_DEVICE,
                     "grouped_fwd_split_noalloc: no device address for the library scratch");
  return grouped_fwd(a, lda, a_scales, ldas, w, w_group_stride, ldw, w_scales, ws_group_stride,
                     ldws, group_ends, num_groups, M, N, K, out, ldo, out_dtype, ws, stream);
}

static int grouped_wgrad(const void* go_t, int64_t ldgo, const void* go_scales_t, int64_t ldgos,
                         const void* ia_t, int64_t ldia, const void* ia_scales_t, int64_t ldias,
                         const int32_t* group_ends, int64_t num_groups, int64_t M, int64_t N,
                         int64_t K, void* dw, int64_t ldw_e, int64_t ldw_n, int out_dtype,
                         int64_t split_tokens, void* workspace, void* stream) {
  if (out_dtype != MXGG_OUT_BF16 && out_dtype != MXGG_OUT_F32)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_wgrad: unknown out_dtype %d", out_dtype);
  if (M < 0 || N < 0 || K < 0)
    return set_error(MXGG_ERR_SHAPE, "grouped_wgrad: negative size");
  if (num_groups < 1 || num_groups > kMaxGroupsAbi)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_wgrad: num_groups=%lld outside [1, %lld]",
                     (long long)num_groups, (long long)kMaxGroupsAbi);
  if (!group_ends)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_wgrad: group_ends is required");
  const bool scaled = go_scales_t != nullptr;
  if ((go_scales_t == nullptr) != (ia_scales_t == nullptr))
    return set_error(MXGG_ERR_INVALID_ARGUMENT,
                     "grouped_wgrad: go_scales_t and ia_scales_t must both be given or both NULL");
  if (M % 32 != 0)
    return set_error(MXGG_ERR_SHAPE, "grouped_wgrad: token count M=%lld not a multiple of 32",
                     (long long)M);
  if (split_tokens < 0 || split_tokens % 128 != 0 || split_tokens > INT32_MAX)
    return set_error(MXGG_ERR_INVALID_ARGUMENT,
                     "grouped_wgrad: split_tokens=%lld must be 0 or a positive multiple of 128",
                     (long long)split_tokens);
  if (split_tokens > 0 && out_dtype != MXGG_OUT_F32 && workspace == nullptr)
    return set_error(MXGG_ERR_UNSUPPORTED,
                     "grouped_wgrad: split-K accumulates with fp32 atomics (out_dtype F32 only)");
  if (N == 0 || K == 0) return MXGG_OK;
  if (!dw) return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_wgrad: null dw");
  if (M > 0 && (!go_t || !ia_t))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_wgrad: null operand");
  if (ldgo < M || ldia < M || (scaled && (ldgos < N || ldias < K)))
    return set_error(MXGG_ERR_SHAPE,
                     "grouped_wgrad: leading dimension smaller than the row (block-major scales: "
                     "ldgos >= N, ldias >= K)");
  if (scaled && ((reinterpret_cast<uintptr_t>(go_scales_t) |
                  reinterpret_cast<uintptr_t>(ia_scales_t)) % 4 != 0 ||
                 ldgos % 4 != 0 || ldias % 4 != 0))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "grouped_wgrad: scale bases and strides must be multiples of 4");
  if (scaled && ((M / 32) * ldgos > kMaxBufferBytes || (M / 32) * ldias > kMaxBufferBytes))
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_wgrad: scale array larger than 2 GiB");
  // No tokens (M == 0): the operands are never read and every expert's dW is
  // written as zeros, so their layout does not matter.
  if (M > 0 && ((go_t && !aligned16(go_t)) || (ia_t && !aligned16(ia_t)) || ldgo % 16 != 0 ||
                ldia % 16 != 0))
    return set_error(MXGG_ERR_ALIGNMENT,
                     "grouped_wgrad: operands must be 16-byte aligned with ld % 16 == 0");
  const int esz = out_dtype == MXGG_OUT_F32 ? 4 : 2;
  // Rows of any K: the epilogues store whole 4-element vectors only inside a
  // row and the rest element by element, so only the base and the strides
  // (checked below) need vector alignment.
  if ((reinterpret_cast<uintptr_t>(dw) % (esz * 4)) != 0)
    return set_error(MXGG_ERR_ALIGNMENT, "grouped_wgrad: dw must be aligned to 4 elements");
  if (ldw_n < K || ldw_e < 0 || (num_groups > 1 && ldw_e < (N - 1) * ldw_n + K))
    return set_error(MXGG_ERR_SHAPE,
                     "grouped_wgrad: dW strides (expert %lld, row %lld) overlap an [N=%lld, "
                     "K=%lld] block",
                     (long long)ldw_e, (long long)ldw_n, (long long)N, (long long)K);
  if (ldw_n % 4 != 0 || ldw_e % 4 != 0)
    return set_error(MXGG_ERR_ALIGNMENT, "grouped_wgrad: dW strides must be multiples of 4");
  if ((N - 1) * ldgo + M > kMaxBufferBytes || (K - 1) * ldia + M > kMaxBufferBytes)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_wgrad: operand larger than 2 GiB");
  if (ldgo > kMaxRowStride || ldia > kMaxRowStride)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_wgrad: row stride above 8 MiB");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "grouped_wgrad: dimension above 2^31");
  WgradArgs args;
  args.go = static_cast<const uint8_t*>(go_t);
  args.gos = static_cast<const uint8_t*>(go_scales_t);
  args.ia = static_cast<const uint8_t*>(ia_t);
  args.ias = static_cast<const uint8_t*>(ia_scales_t);
  args.group_ends = group_ends;
  args.dw = dw;
  args.ldgo = ldgo;
  args.ldgos = scaled ? ldgos : 0;
  args.ldia = ldia;
  args.ldias = scaled ? ldias : 0;
  args.ldw_e = ldw_e;
  args.ldw_n = ldw_n;
  args.M = (int32_t)M;
  args.N = (int32_t)N;
  args.K = (int32_t)K;
  args.E = (int32_t)num_groups;
  args.split = (int32_t)split_tokens;
  args.out_f32 = out_dtype == MXGG_OUT_F32;
  args.scaled = scaled;
  args.split_ws = static_cast<float*>(workspace);
  return check_launch(launch_grouped_wgrad(args, static_cast<hipStream_t>(stream)),
                      "grouped_wgrad");
}

int mxgg_grouped_wgrad(const void* go_t, int64_t ldgo, const void* go_scales_t, int64_t ldgos,
                       const void* ia_t, int64_t ldia, const void* ia_scales_t, int64_t ldias,
                       const int32_t* group_ends, int64_t num_groups, int64_t M, int64_t N,
                       int64_t K, void* dw, int out_dtype, int64_t split_tokens, void* stream) {
  return grouped_wgrad(go_t, ldgo, go_scales_t, ldgos, ia_t, ldia, ia_scales_t, ldias,
                       group_ends, num_groups, M, N, K, dw, N * K, K, out_dtype, split_tokens,
                       nullptr, stream);
}

int64_t mxgg_grouped_wgrad_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t num_groups,
                                           int64_t split_tokens) {
  if (M < 0 || N < 0 || K < 0 || num_groups < 1 || split_tokens < 128) return -1;
  return wgrad_split_workspace_bytes(M, N, K, num_groups, split_tokens);
}

static int grouped_wgrad_split(const void* go_t, int64_t ldgo, const void* go_scales_t,
                               int64_t ldgos, const void* ia_t, int64_t ldia,
                               const void* ia_scales_t, int64_t ldias,
                               const int32_t* group_ends, int64_t num_groups, int64_t M,
                               int64_t N, int64_t K, void* dw, int64_t ldw_e, int64_t ldw_n,
                               int out_dtype, int64_t split_tokens, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  if (split_tokens <= 0 || split_tokens % 128 != 0 || split_tokens > INT32_MAX)
    return set_error(MXGG_ERR_INVALID_ARGUMENT,
                     "grouped_wgrad_split: split_tokens=%lld must be a positive multiple of 128",
                     (long long)split_tokens);
  if (!workspace)
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "grouped_wgrad_split: null workspace");
  if (num_groups >= 1 && num_groups <= kMaxGroupsAbi && M >= 0 && N >= 0 && K >= 0 &&
      workspace_bytes < wgrad_split_workspace_bytes(M, N, K, num_groups, split_tokens))
    return set_error(MXGG_ERR_SHAPE, "grouped_wgrad_split: workspace_bytes=%lld < %lld",
                     (long long)workspace_bytes,
                     (long long)wgrad_split_workspace_bytes(M, N, K, num_groups, split_tokens));
  if (!aligned16(workspace))
    return set_error(MXGG_ERR_ALIGNMENT, "grouped_wgrad_split: workspace must be 16-byte aligned");
  return grouped_wgrad(go_t, ldgo, go_scales_t, ldgos, ia_t, ldia, ia_scales_t, ldias,
                       group_ends, num_groups, M, N, K, dw, ldw_e, ldw_n, out_dtype, split_tokens,
                       workspace, stream);
}

int mxgg_grouped_wgrad_split(const void* go_t, int64_t ldgo, const void* go_scales_t,
                             int64_t ldgos, const void* ia_t, int64_t ldia,
                             const void* ia_scales_t, int64_t ldias, const int32_t* group_ends,
                             int64_t num_groups, int64_t M, int64_t N, int64_t K, void* dw,
                             int out_dtype, int64_t split_tokens, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  return grouped_wgrad_split(go_t, ldgo, go_scales_t, ldgos, ia_t, ldia, ia_scales_t, ldias,
                             group_ends, num_groups, M, N, K, dw, N * K, K, out_dtype,
                             split_tokens, workspace, workspace_bytes, stream);
}

int mxgg_grouped_wgrad_strided(const void* go_t, int64_t ldgo, const void* go_scales_t,
                               int64_t ldgos, const void* ia_t, int64_t ldia,
                               const void* ia_scales_t, int64_t ldias,
                               const int32_t* group_ends, int64_t num_groups, int64_t M,
                               int64_t N, int64_t K, void* dw, int64_t ld_dw_expert,
                               int64_t ld_dw_row, int out_dtype, int64_t split_tokens,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace == nullptr)
    return grouped_wgrad(go_t, ldgo, go_scales_t, ldgos, ia_t, ldia, ia_scales_t, ldias,
                         group_ends, num_groups, M, N, K, dw, ld_dw_expert, ld_dw_row, out_dtype,
                         split_tokens, nullptr, stream);
  return grouped_wgrad_split(go_t, ldgo, go_scales_t, ldgos, ia_t, ldia, ia_scales_t, ldias,
                             group_ends, num_groups, M, N, K, dw, ld_dw_expert, ld_dw_row,
                             out_dtype, split_tokens, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Token routing.
// ---------------------------------------------------------------------------
// Argument checks shared by both route-plan entries (0 when valid).
static int check_route_plan(const int32_t* expert_idx, int64_t tokens, int64_t topk,
                            int64_t num_experts, int64_t pad_multiple, int64_t rows_cap,
                            const int32_t* perm, const int32_t* src, const int32_t* group_ends,
                            const int32_t* counts) {
  if (tokens < 0 || topk < 1 || rows_cap < 0)
    return set_error(MXGG_ERR_SHAPE, "route_plan: tokens=%lld, topk=%lld, rows_cap=%lld",
                     (long long)tokens, (long long)topk, (long long)rows_cap);
  if (num_experts < 1 || num_experts > kMaxGroupsAbi)
    return set_error(MXGG_ERR_UNSUPPORTED, "route_plan: num_experts=%lld outside [1, %lld]",
                     (long long)num_experts, (long long)kMaxGroupsAbi);
  if (pad_multiple < 1 || pad_multiple > 1024)
    return set_error(MXGG_ERR_UNSUPPORTED, "route_plan: pad_multiple=%lld outside [1, 1024]",
                     (long long)pad_multiple);
  if (tokens > INT32_MAX / topk)
    return set_error(MXGG_ERR_UNSUPPORTED, "route_plan: tokens * topk above 2^31");
  const int64_t n = tokens * topk;
  const int64_t need = n + num_experts * (pad_multiple - 1);
  if (rows_cap < need)
    return set_error(MXGG_ERR_SHAPE, "route_plan: rows_cap=%lld < tokens*topk + E*(pad-1) = %lld",
                     (long long)rows_cap, (long long)need);
  if (rows_cap > INT32_MAX)
    return set_error(MXGG_ERR_UNSUPPORTED, "route_plan: rows_cap above 2^31");
  if (!group_ends || !counts || (n > 0 && (!expert_idx || !perm)) || (rows_cap > 0 && !src))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "route_plan: null pointer");
  return MXGG_OK;
}

int mxgg_route_plan(const int32_t* expert_idx, int64_t tokens, int64_t topk, int64_t num_experts,
                    int64_t pad_multiple, int64_t rows_cap, int32_t* perm, int32_t* src,
                    int32_t* group_ends, int32_t* counts, void* stream) {
  const int rc = check_route_plan(expert_idx, tokens, topk, num_experts, pad_multiple, rows_cap,
                                  perm, src, group_ends, counts);
  if (rc != MXGG_OK) return rc;
  return check_launch(launch_route_plan(expert_idx, tokens * topk, (int)num_experts,
                                        (int)pad_multiple, rows_cap, perm, src, group_ends, counts,
                                        static_cast<hipStream_t>(stream)),
                      "route_plan");
}

int64_t mxgg_route_plan_workspace_bytes(int64_t tokens, int64_t topk, int64_t num_experts) {
  if (tokens < 0 || topk < 1 || num_experts < 1 || num_experts > kMaxGroupsAbi ||
      tokens > INT32_MAX / topk)
    return -1;
  return route_plan_blocks(tokens * topk) * num_experts * 4;
}

int mxgg_route_plan_ws(const int32_t* expert_idx, int64_t tokens, int64_t topk,
                       int64_t num_experts, int64_t pad_multiple, int64_t rows_cap, int32_t* perm,
                       int32_t* src, int32_t* group_ends, int32_t* counts, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  const int rc = check_route_plan(expert_idx, tokens, topk, num_experts, pad_multiple, rows_cap,
                                  perm, src, group_ends, counts);
  if (rc != MXGG_OK) return rc;
  const int64_t need = mxgg_route_plan_workspace_bytes(tokens, topk, num_experts);
  if (workspace_bytes < need)
    return set_error(MXGG_ERR_SHAPE, "route_plan_ws: workspace of %lld bytes, %lld needed",
                     (long long)workspace_bytes, (long long)need);
  if (need > 0 && (!workspace || reinterpret_cast<uintptr_t>(workspace) % 4 != 0))
    return set_error(workspace ? MXGG_ERR_ALIGNMENT : MXGG_ERR_INVALID_ARGUMENT,
                     "route_plan_ws: the workspace must be a 4-byte aligned device buffer");
  return check_launch(launch_route_plan_blocks(expert_idx, tokens * topk, (int)num_experts,
                                               (int)pad_multiple, rows_cap, perm, src, group_ends,
                                               counts, static_cast<int32_t*>(workspace),
                                               static_cast<hipStream_t>(stream)),
                      "route_plan_ws");
}

// Rows of 16-byte bf16 chunks: cols % 8 == 0, 16-byte aligned bases and strides.
static int check_rows(const char* what, const void* a, int64_t lda, const void* b, int64_t ldb,
                      int64_t cols) {
  if (cols < 0 || cols % 8 != 0)
    return set_error(MXGG_ERR_SHAPE, "%s: cols=%lld is not a non-negative multiple of 8", what,
                     (long long)cols);
  if (cols > INT32_MAX) return set_error(MXGG_ERR_UNSUPPORTED, "%s: cols above 2^31", what);
  if (lda < cols || ldb < cols)
    return set_error(MXGG_ERR_SHAPE, "%s: leading dimension smaller than the row", what);
  if ((a && !aligned16(a)) || (b && !aligned16(b)) || lda % 8 != 0 || ldb % 8 != 0)
    return set_error(MXGG_ERR_ALIGNMENT,
                     "%s: rows 16-byte aligned with leading dimensions multiples of 8", what);
  return MXGG_OK;
}

int mxgg_gather_rows(const void* x, int64_t tokens, int64_t cols, int64_t ldx, const int32_t* src,
                     int64_t topk, const float* row_scale, int64_t rows, void* out, int64_t ldo,
                     void* stream) {
  if (tokens < 0 || rows < 0 || topk < 1)
    return set_error(MXGG_ERR_SHAPE, "gather_rows: tokens=%lld, rows=%lld, topk=%lld",
                     (long long)tokens, (long long)rows, (long long)topk);
  const int st = check_rows("gather_rows", x, ldx, out, ldo, cols);
  if (st != MXGG_OK) return st;
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !out || (tokens > 0 && !x))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "gather_rows: null pointer");
  if (topk > INT32_MAX || rows > kMaxWaveRows)
    return set_error(MXGG_ERR_UNSUPPORTED, "gather_rows: rows above %lld", (long long)kMaxWaveRows);
  return check_launch(launch_gather_rows(static_cast<const uint16_t*>(x), ldx, tokens, src,
                                         (int)topk, row_scale, rows, cols,
                                         static_cast<uint16_t*>(out), ldo,
                                         static_cast<hipStream_t>(stream)),
                      "gather_rows");
}

int mxgg_gather_quant_dual(const void* x, int64_t tokens, int64_t cols, int64_t ldx,
                           const int32_t* src, int64_t topk, const float* row_scale, int64_t rows,
                           const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap,
                           void* q, int64_t ldq, void* scales, int64_t lds, void* qt, int64_t ldqt,
                           void* scales_t, int64_t ldst, int scale_layout,
                           int32_t* group_ends_pad, int scale_mode, void* stream) {
  if (tokens < 0 || topk < 1 || topk > INT32_MAX)
    return set_error(MXGG_ERR_SHAPE, "gather_quant_dual: tokens=%lld, topk=%lld",
                     (long long)tokens, (long long)topk);
  const int st = check_dual("gather_quant_dual", x != nullptr || tokens == 0, rows, cols, ldx,
                            group_ends, num_groups, rows_pad_cap, q, ldq, scales, lds, qt, ldqt,
                            scales_t, ldst, scale_layout, group_ends_pad, scale_mode, x);
  if (st != MXGG_OK || cols == 0 || rows_pad_cap == 0) return st;
  if (rows > 0 && !src) return set_error(MXGG_ERR_INVALID_ARGUMENT, "gather_quant_dual: null src");
  return check_launch(
      launch_gather_quant_dual(static_cast<const uint16_t*>(x), tokens, ldx, src, (int)topk,
                               row_scale, rows, cols, group_ends, group_ends ? num_groups : 1,
                               rows_pad_cap, static_cast<uint8_t*>(q), ldq,
                               static_cast<uint8_t*>(scales), lds, static_cast<uint8_t*>(qt), ldqt,
                               static_cast<uint8_t*>(scales_t), ldst, scale_layout, group_ends_pad,
                               scale_mode, static_cast<hipStream_t>(stream)),
      "gather_quant_dual");
}

int mxgg_gather_quant_dim0(const void* x, int64_t tokens, int64_t cols, int64_t ldx,
                           const int32_t* src, int64_t topk, int64_t rows, void* q, int64_t ldq,
                           void* scales, int64_t lds, int scale_layout, int scale_mode,
                           void* stream) {
  if (tokens < 0 || topk < 1 || topk > INT32_MAX)
    return set_error(MXGG_ERR_SHAPE, "gather_quant_dim0: tokens=%lld, topk=%lld",
                     (long long)tokens, (long long)topk);
  // x may be empty (no tokens): the check then needs a stand-in address
  const void* xv = (x == nullptr && tokens == 0) ? q : x;
  const int st = check_dim0("gather_quant_dim0", xv, rows, cols, ldx, q, ldq, scales, lds,
                            scale_layout, scale_mode);
  if (st != MXGG_OK || rows == 0 || cols == 0) return st;
  if (!src) return set_error(MXGG_ERR_INVALID_ARGUMENT, "gather_quant_dim0: null src");
  // the column blocks of 512 form the grid's y dimension
  if ((cols + 511) / 512 > 65535)
    return set_error(MXGG_ERR_UNSUPPORTED, "gather_quant_dim0: cols=%lld above 65535 * 512",
                     (long long)cols);
  return check_launch(
      launch_gather_quant_dim0(static_cast<const uint16_t*>(x), tokens, ldx, src, (int)topk, rows,
                               cols, static_cast<uint8_t*>(q), ldq, static_cast<uint8_t*>(scales),
                               lds, scale_layout, scale_mode, static_cast<hipStream_t>(stream)),
      "gather_quant_dim0");
}

int mxgg_combine(const void* y, int64_t rows, int64_t cols, int64_t ldy, const int32_t* perm,
                 const float* scores, int64_t tokens, int64_t topk, void* out, int64_t ldo,
                 void* stream) {
  if (rows < 0 || tokens < 0 || topk < 1 || topk > INT32_MAX)
    return set_error(MXGG_ERR_SHAPE, "combine: rows=%lld, tokens=%lld, topk=%lld",
                     (long long)rows, (long long)tokens, (long long)topk);
  const int st = check_rows("combine", y, ldy, out, ldo, cols);
  if (st != MXGG_OK) return st;
  if (tokens == 0 || cols == 0) return MXGG_OK;
  if (!perm || !out || (rows > 0 && !y))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "combine: null pointer");
  if (tokens > kMaxWaveRows)
    return set_error(MXGG_ERR_UNSUPPORTED, "combine: tokens above %lld", (long long)kMaxWaveRows);
  return check_launch(launch_combine(static_cast<const uint16_t*>(y), ldy, rows, perm, scores,
                                     tokens, (int)topk, cols, static_cast<uint16_t*>(out), ldo,
                                     static_cast<hipStream_t>(stream)),
                      "combine");
}

int mxgg_combine_score_grad(const void* grad_out, int64_t ldg, const void* y, int64_t rows,
                            int64_t cols, int64_t ldy, const int32_t* perm, int64_t tokens,
                            int64_t topk, float* grad_scores, void* stream) {
  if (rows < 0 || tokens < 0 || topk < 1 || topk > INT32_MAX)
    return set_error(MXGG_ERR_SHAPE, "combine_score_grad: rows=%lld, tokens=%lld, topk=%lld",
                     (long long)rows, (long long)tokens, (long long)topk);
  const int st = check_rows("combine_score_grad", grad_out, ldg, y, ldy, cols);
  if (st != MXGG_OK) return st;
  if (tokens == 0) return MXGG_OK;
  if (!perm || !grad_scores || (cols > 0 && (!grad_out || (rows > 0 && !y))))
    return set_error(MXGG_ERR_INVALID_ARGUMENT, "combine_score_grad: null pointer");
  if (tokens > kMaxWaveRows)
    return set_error(MXGG_ERR_UNSUPPORTED, "combine_score_grad: tokens above %lld",
                     (long long)kMaxWaveRows);
  return check_launch(
      launch_combine_score_grad(static_cast<const uint16_t*>(grad_out), ldg,
                                static_cast<const uint16_t*>(y), ldy, rows, perm, tokens,
                                (int)topk, cols, grad_scores, static_cast<hipStream_t>(stream)),
      "combine_score_grad");
}

}  // extern "C"
