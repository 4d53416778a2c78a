/*
 * mx_oracle.c — CPU restatement of the MXFP8 arithmetic on the reference's hot
 * path.  TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker; never linked into libmxgg.so.
 *
 * What it restates (reference citations are /root/reference paths):
 *   - E8M0 meaning 2^(b-127), 0xFF = NaN, block of 32 along the contraction
 *     dimension: SCALE_FINDINGS.md:14-54, scale_correctness.py:30-34.
 *   - Block quantisation along K with a per-(row, block) scale:
 *     scale_correctness.py:91-106 (known-scale construction) and the recipe
 *     "mxfp8_rceil" selected by the trainer integration (port_mxfp8.py:178,
 *     207-213).  The scale rules are those of torchao's to_mx() (third-party,
 *     torchao fork indianspeedster/ao @ rocm-mxfp8-optimizations-v2, no pinned
 *     commit; not present in /root/reference):
 *       RCEIL: b = clamp(ceil(log2(amax/448)), -127, 127) + 127;
 *              payload = clamp(x * (b == 0 ? 1 : 2^(127-b)), +-448)
 *       FLOOR: b = clamp(floor(log2(amax)) - 8, -127, 128) + 127;
 *              payload = clamp(x / max(2^(b-127), 2^-126), +-448)
 *       NaN anywhere in the block -> b = 0xFF.
 *   - Payload cast: round-to-nearest-even to OCP float8 e4m3fn, as
 *     torch's .to(torch.float8_e4m3fn) (e2e_bench.py:35-40); NaN -> 0x7F|sign.
 *   - Token-axis (dim1) quantisation with per-group restart and 32-padding:
 *     the transposed, token-contiguous wgrad operands of wgrad_fused.py:35-39,
 *     48-62 without the equal-group assumption.
 *
 * Parity unpinned (no reference vector or fixture decides them; the oracle
 * keeps the closed forms above): the byte of an infinite amax (RCEIL 254,
 * FLOOR 247), of an all-zero block (0), and the RCEIL payload multiplier 1
 * for scale byte 0 (blocks with amax < 448 * 2^-127).  Every other rule is
 * checked against torch's e4m3 cast, brute force and the reference's
 * known-answer vectors (tests/test_oracle.py).
 *
 * The implementation deliberately differs from the GPU kernels: e4m3 rounding
 * is a nearest-value search over the decoded code table, and the scale
 * exponents come from double-precision frexp(), not from bit tricks.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define MXO_RCEIL 0
#define MXO_FLOOR 1

static double g_e4m3_pos[127]; /* value of positive finite code c, c = 0..126 */
static int g_table_ready = 0;

/* OCP e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits; 0x7F/0xFF NaN,
 * no infinities; exponent field 0 is subnormal: m * 2^-9. */
double mxo_e4m3_decode(uint8_t code) {
  const int s = code >> 7;
  const int e = (code >> 3) & 15;
  const int m = code & 7;
  double v;
  if ((code & 0x7F) == 0x7F) return NAN;
  if (e == 0) v = ldexp((double)m, -9);
  else v = ldexp(1.0 + m / 8.0, e - 7);
  return s ? -v : v;
}

static void init_table(void) {
  if (g_table_ready) return;
  for (int c = 0; c < 127; ++c) g_e4m3_pos[c] = mxo_e4m3_decode((uint8_t)c);
  g_table_ready = 1;
}

/* Round-to-nearest-even onto the e4m3fn grid, without saturation: like torch,
 * a value that rounds above 448 (|v| > 464, the midpoint to the next binade
 * step) becomes NaN. */
uint8_t mxo_e4m3_encode(double v) {
  init_table();
  if (isnan(v)) return (uint8_t)(0x7F | (signbit(v) ? 0x80 : 0));
  const uint8_t s = signbit(v) ? 0x80 : 0;
  const double a = fabs(v);
  if (a > 464.0) return (uint8_t)(s | 0x7F);
  if (a >= 448.0) return (uint8_t)(s | 0x7E);
  /* largest code with value <= a */
  int lo = 0, hi = 126;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (g_e4m3_pos[mid] <= a) lo = mid; else hi = mid - 1;
  }
  int c = lo;
  if (g_e4m3_pos[c] != a && c < 126) {
    const double dlo = a - g_e4m3_pos[c];
    const double dhi = g_e4m3_pos[c + 1] - a;
    if (dhi < dlo || (dhi == dlo && ((c + 1) % 2 == 0))) c = c + 1;
  }
  return (uint8_t)(s | c);
}

static double bf16_to_double(uint16_t h) {
  union { uint32_t u; float f; } x;
  x.u = (uint32_t)h << 16;
  return (double)x.f;
}

/* E8M0 byte for a block whose max |x| is amax (amax >= 0 or NaN). */
uint8_t mxo_e8m0(double amax, int mode) {
  if (isnan(amax)) return 0xFF;
  if (mode == MXO_RCEIL) {
    if (amax == 0.0) return 0;               /* ceil(log2 0) = -inf -> clamp -127 */
    if (isinf(amax)) return 254;             /* +inf -> clamp +127 */
    const double d = amax / 448.0;           /* exact power of two stays exact */
    int e;
    const double f = frexp(d, &e);           /* d = f * 2^e, f in [0.5, 1) */
    int c = (f == 0.5) ? e - 1 : e;          /* ceil(log2(d)) */
    if (c < -127) c = -127;
    if (c > 127) c = 127;
    return (uint8_t)(c + 127);
  } else {
    int fl;
    if (amax == 0.0) return 0;
    if (isinf(amax)) fl = 128;               /* exponent field of +inf */
    else {
      int e;
      frexp(amax, &e);
      fl = e - 1;                            /* floor(log2(amax)) */
      if (amax < ldexp(1.0, -126)) fl = -127; /* fp32 subnormal: exponent field 0 */
    }
    int c = fl - 8;
    if (c < -127) c = -127;
    if (c > 128) c = 128;
    return (uint8_t)(c + 127);
  }
}

/* Payload code of one element given its block's scale byte. */
uint8_t mxo_payload(double x, uint8_t b, int mode) {
  double y;
  if (isnan(x)) return mxo_e4m3_encode(x);
  if (mode == MXO_RCEIL) {
    y = (b == 0) ? x : ldexp(x, 127 - (int)b);
  } else {
    if (b == 255) {                          /* divide by +inf */
      if (isinf(x)) return 0x7F;             /* inf/inf: a fresh (positive) NaN */
      y = signbit(x) ? -0.0 : 0.0;
    } else {
      y = ldexp(x, 127 - (b < 1 ? 1 : (int)b));
    }
  }
  if (y > 448.0) y = 448.0;
  if (y < -448.0) y = -448.0;
  return mxo_e4m3_encode(y);
}

/* Quantise one block of n <= 32 bf16 values (missing values count as +0). */
static uint8_t quant_block(const double* v, int n, uint8_t* out, int mode) {
  double amax = 0.0;
  int has_nan = 0;
  for (int i = 0; i < n; ++i) {
    if (isnan(v[i])) has_nan = 1;
    else if (fabs(v[i]) > amax) amax = fabs(v[i]);
  }
  const uint8_t b = mxo_e8m0(has_nan ? NAN : amax, mode);
  for (int i = 0; i < n; ++i) out[i] = mxo_payload(v[i], b, mode);
  return b;
}

/* dim0: x bf16 [rows, cols] row-major -> q [rows, cols], s [rows, cols/32]. */
void mxo_quant_dim0(const uint16_t* x, int64_t rows, int64_t cols, uint8_t* q, uint8_t* s,
                    int mode) {
  double v[32];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t cb = 0; cb < cols / 32; ++cb) {
      for (int i = 0; i < 32; ++i) v[i] = bf16_to_double(x[r * cols + cb * 32 + i]);
      s[r * (cols / 32) + cb] = quant_block(v, 32, q + r * cols + cb * 32, mode);
    }
}

/* dim1: x bf16 [rows, cols]; groups by cumulative ends (ends == NULL: one
 * group of all rows).  Output qt [cols, cap] and st [cols, cap/32], group g
 * occupying padded columns [pend[g-1], pend[g]) with pend the cumulative sum of
 * 32*ceil(size/32); the tail of a group and every column past the last group
 * hold zeros, scale computed as for an all-zero block. */
void mxo_quant_dim1(const uint16_t* x, int64_t rows, int64_t cols, const int32_t* ends,
                    int64_t E, int64_t cap, uint8_t* qt, uint8_t* st, int32_t* ends_pad,
                    int mode) {
  double v[32];
  uint8_t out[32];
  const int64_t groups = ends ? E : 1;
  int64_t pcol = 0;
  int64_t m_prev = 0; /* running maximum of the clamped ends */
  memset(qt, 0, (size_t)(cols * cap));
  for (int64_t g = 0; g < groups; ++g) {
    /* group g = [m[g-1], m[g]), m[g] = max(m[g-1], clamp(ends[g], 0, rows)) */
    const int64_t beg = m_prev;
    int64_t end = ends ? ends[g] : rows;
    end = end < 0 ? 0 : (end > rows ? rows : end);
    if (end < beg) end = beg;
    m_prev = end;
    const int64_t size = end - beg;
    const int64_t nblk = (size + 31) / 32;
    for (int64_t c = 0; c < cols; ++c)
      for (int64_t b = 0; b < nblk; ++b) {
        for (int i = 0; i < 32; ++i) {
          const int64_t t = beg + b * 32 + i;
          v[i] = t < end ? bf16_to_double(x[t * cols + c]) : 0.0;
        }
        const uint8_t s = quant_block(v, 32, out, mode);
        memcpy(qt + c * cap + pcol + b * 32, out, 32);
        st[c * (cap / 32) + (pcol / 32) + b] = s;
      }
    pcol += nblk * 32;
    if (ends_pad) ends_pad[g] = (int32_t)pcol;
  }
  /* columns past the padded total: zero blocks */
  for (int64_t c = 0; c < cols; ++c)
    for (int64_t p = pcol; p < cap; p += 32) st[c * (cap / 32) + p / 32] = mxo_e8m0(0.0, mode);
}

/* Dequantise [rows, cols] payload + [rows, cols/32] scales into doubles. */
void mxo_dequant(const uint8_t* q, const uint8_t* s, int64_t rows, int64_t cols, int64_t ldq,
                 int64_t lds, double* out) {
  init_table();
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const uint8_t b = s ? s[r * lds + c / 32] : 127;
      const double sc = (b == 255) ? NAN : ldexp(1.0, (int)b - 127);
      out[r * cols + c] = mxo_e4m3_decode(q[r * ldq + c]) * sc;
    }
}
