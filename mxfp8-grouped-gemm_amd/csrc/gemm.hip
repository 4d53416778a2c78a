// MXFP8 grouped GEMM kernels for gfx950 (CDNA4) on v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Both kernels compute tiles of
//   D[p][q] = sum_k P[p][k] * 2^(sP[k/32][p]-127) * Q[q][k] * 2^(sQ[k/32][q]-127)
// where P and Q are row-major e4m3 operands contiguous along the contraction
// dimension k and the E8M0 scales are stored block-major (one row of bytes per
// 32-deep k-block, indexed by operand row).  P feeds the MFMA "A" source and Q
// the "B" source; each lane ends up holding runs of 4 consecutive P indices
// (one from each of its 4 MFMA blocks along P) for one Q index, so the
// output's contiguous dimension is the P index.
//
//   forward : P = W[g] (rows n), Q = X (rows m of group g), k = hidden  -> Y[m][n]
//   wgrad   : P = X^T  (rows k), Q = dY^T (rows n),  k = tokens of g    -> dW[g][n][k]
//
// Tile 256(P) x 256(Q), 256 threads = 4 waves in a 2x2 arrangement, each wave
// 128x128 = 4x4 MFMA 32x32 blocks (256 fp32 accumulators per lane in AGPRs).
// MFMA block i of a wave's 128 rows takes every 4th row (rows 4m+i), so the
// four scale bytes a lane needs for one k-block are adjacent in the
// block-major scale row and arrive with one 32-bit LDS read.
//
// The contraction streams through two LDS stages of 128 (four k-blocks, two
// MFMA k-steps).  A stage holds P and Q (256 rows x 128 B each: every row is
// one whole 128-byte cache line of the operand, 16-byte chunks XOR-swizzled)
// and their 8 scale rows, all written by LDS-DMA (buffer_load ... lds).
// Reading whole lines matters: with 64-byte stages every line crossed the
// L2 -> L1 path twice and the L2 request rate, not the MFMA pipe, set the
// speed.  Each stage has a release barrier (every wave has read the stage into
// registers, so its slot can be refilled with stage s+2) and a publish barrier
// (stage s+1 has landed); the loads are spread one per MFMA, because a DMA
// instruction stalls its wave's issue until the address unit accepts it.
// Persistent grid (one workgroup per CU), tiles dealt round-robin with each XCD
// taking a contiguous slice of every round.
#include <algorithm>
#include <mutex>
#include <vector>

#include "mx_device.h"
#include "mxgg_internal.h"

namespace mxgg {
namespace {

constexpr int kTileP = 256;
constexpr int kTileQ = 256;
constexpr int kStageK = 128;    // contraction elements (bytes) per stage
constexpr int kThreads = 256;
constexpr uint32_t kOpBytes = 256u * kStageK;          // one operand of one stage: 32 KB
constexpr uint32_t kScaleOff = 2u * kOpBytes;          // scale rows after P and Q data
// Scale block b of a stage at kScaleOff + b * kScaleBlk: [P, Q][256] bytes and
// 64 bytes of padding, so that the lanes of blocks 0 and 1 (one half-wave of
// a scale read) fall on different banks.
constexpr uint32_t kScaleBlk = 576;
constexpr uint32_t kStageBytes = kScaleOff + 4u * kScaleBlk;
constexpr uint32_t kOobOffset = 0x80000000u;           // beyond every num_records we create
// Split-K of the forward's last round: at most this many K-ranges per tile;
// workspace = a header (tail tile count, split count, then q0, p0, group
// begin and end of every split tile) and one fp32 256x256 partial per split.
constexpr uint32_t kMaxSplit = 16;
// After at least one full round, the sparse last round is cut into at most
// this many ranges: fewer partials for the reduction to read, and the pieces
// still land on idle units (measured on C2's 16-tile 18th round: +1.2% with
// 8 or 4 ranges, +0.3% with 16).
constexpr uint32_t kMaxSplitTail = 8;
constexpr int64_t kSplitHdrBytes = 16384;
constexpr int64_t kPartialBytes = 256 * 256 * 4;
// Wgrad split with a workspace: header = E, items per expert, tile counts,
// band width, then (expert, first item, chunks) of every rank; partial of
// work item i at kWgHdrBytes + i * kPartialBytes.
constexpr int64_t kWgHdrBytes = 32768;

struct __align__(16) Smem {
  uint8_t ring[2][kStageBytes];
  int32_t sched[kMaxGroups + 1];
  int32_t order[kMaxGroups];
  int32_t scan_tmp[kThreads];
  int32_t chunks[kMaxGroups];      // wgrad: split-K chunks of the expert of each rank
  int32_t items[kMaxGroups + 1];   // wgrad: prefix of work items over ranks
  int32_t gend[kMaxGroups];        // monotone clamped group ends (monotone_ends_to_lds)
};

// Raw 128-bit buffer descriptor (gfx9 layout: base, stride 0, num_records,
// dst_sel/format word).  Offsets at or past num_records read as zero.
typedef int32_t desc_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ desc_t make_desc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  desc_t d;
  d[0] = (int32_t)(uint32_t)a;
  d[1] = (int32_t)((uint32_t)(a >> 32) & 0xFFFFu);
  d[2] = (int32_t)bytes;
  d[3] = 0x00020000;
  return d;
}

// Readable bytes of a block-major scale array with `nblk` block-rows of
// stride `ld` holding `rows` rows: the scale DMA reads whole 4-row dwords.
__device__ __forceinline__ uint32_t scale_extent(int64_t nblk, int64_t ld, int64_t rows) {
  return (uint32_t)((nblk - 1) * ld + ((rows + 3) & ~(int64_t)3));
}

// One operand of a tile.  Rows at or past `rows` are not clamped: their byte
// offsets lie beyond the descriptor's num_records ((rows-1)*ld + K) and read
// as zero.  The C ABI bounds (rows + 256) * ld below 2^32 so these offsets do
// not wrap.
struct Operand {
  desc_t data;    // [rows][ld] e4m3
  desc_t scale;   // [k-blocks][lds] E8M0, block-major
  uint32_t ld;    // bytes per data row
  uint32_t lds;   // bytes per scale block-row (multiple of 4)
  uint32_t row0;  // first operand row of this tile (multiple of 4)
  // Operand row of tile row 128, minus row0: 128 for a plain tile of 256
  // consecutive rows; F for the gate+up tile of the fused SwiGLU forward
  // (tile rows 0..127 = gate rows, 128..255 = the matching up rows F later).
  uint32_t hi;
};

// Cache-policy operand of the buffer store builtins: the nontemporal bit.
constexpr int kCacheNT = 2;

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t wave_id() {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Byte offset of a __shared__ object inside the workgroup's LDS allocation.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)((const lds_void_t*)p);
}

// 16-byte chunk swizzle inside a 128-byte LDS slot.  gfx950 serves a
// ds_read_b128 one half-wave (32 lanes, 512 B) at a time over 64 four-byte
// banks; it runs at full rate when every bank holds at most two of the
// half-wave's dwords.  A half-wave reads one chunk from each of 32 consecutive
// slots; the bank quad of (slot s, chunk c) is 8*(s mod 2) + (c ^ swz(s)), and
// with swz(s) = (s/2) mod 8 the 16 quads are each hit exactly twice.
__device__ __forceinline__ uint32_t swz(uint32_t s) { return (s >> 1) & 7u; }

// Wait for this wave's DMA except the youngest `N` instructions and for all
// of its LDS reads, then the workgroup barrier.  Written as assembly so the
// compiler's waitcnt pass can neither relax nor move it (it does not see the
// DMA, and would drop the lgkmcnt part for reads whose results are only used
// after the barrier).
template <int N>
__device__ __forceinline__ void wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// LDS-DMA issued from inline assembly: M0 holds the wave's LDS destination,
// each lane its byte offset into the buffer.  The compiler does not track
// these loads, so it inserts no wait for them in front of LDS reads of the
// other stage; every consumer waits explicitly in wait_barrier().
// M0 is reserved by the compiler, which warns about the clobber; on gfx950 it
// only uses M0 for LDS-DMA, GWS and message instructions, none of which it
// emits in these kernels (the generated code writes M0 only here).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// soff: a wave-uniform byte offset added in the instruction's scalar offset
// field.  The buffer range check covers voff + soff (measured on gfx950: a
// scalar offset alone past num_records reads zero), so a per-load row step
// can ride there instead of costing a vector add per load.
__device__ __forceinline__ void dma_x4(const desc_t& d, uint32_t lds_addr, uint32_t voff,
                                       uint32_t soff = 0) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds"
      :
      : "s"(lds_addr), "v"(voff), "s"(d), "s"(soff)
      : "memory", "m0");
}
__device__ __forceinline__ void dma_x1(const desc_t& d, uint32_t lds_addr, uint32_t voff,
                                       uint32_t soff = 0) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dword %1, %2, %3 offen lds"
      :
      : "s"(lds_addr), "v"(voff), "s"(d), "s"(soff)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// Per-thread state of the global -> LDS stream for one tile.
//  Data: wave w's i-th load (i = 0..7) fills LDS bytes [4096i + 1024w, +1024)
//  of an operand, lane l writing 16 B at +16l: slot s = 32i + 8w + l/8 at
//  physical chunk l%8, so the lane fetches logical chunk (l%8) ^ swz(s) of
//  tile row 128(i/4) + 4(8w + l/8) + i%4 (slots 128a + 32b + c hold rows
//  128a + 4c + b).  Eight lanes cover one
//  128-byte line.  swz(s) = (4w + l/16) mod 8 does not depend on i, and the
//  row moves by a lane-independent amount from load to load, so the lane keeps
//  one base offset per operand and adds a uniform step.  Chunks outside
//  [klo, kend) are fetched from an out-of-range offset and land as zeros.
//  Scales: wave w copies block k0/32 + w of both operands: 256 rows = 64 lanes
//  x 4 bytes in row order.  A block outside [klo, kend) lands as zeros (scale
//  2^-127 on zero payload).
template <bool SCALED, bool MASK = false>
struct Stream {
  uint32_t vp, vq;   // lane offset of load 0 without k0
  uint32_t kcol;     // lane's chunk column within a stage (bytes)
  uint32_t sp, sq;   // lane offset of its scale dword within a block-row
  uint32_t klo, kend;

  __device__ __forceinline__ void init(const Operand& P, const Operand& Q, uint32_t lo,
                                       uint32_t hi) {
    klo = lo;
    kend = hi;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = wave_id();
    kcol = 16u * ((lane & 7u) ^ ((4u * wave + (lane >> 4)) & 7u));
    const uint32_t r = 4u * (8u * wave + (lane >> 3));
    vp = (P.row0 + r) * P.ld + kcol;
    vq = (Q.row0 + r) * Q.ld + kcol;
    if (SCALED) {
      sp = P.row0 + 4u * lane + (lane >= 32u ? P.hi - 128u : 0u);
      sq = Q.row0 + 4u * lane + (lane >= 32u ? Q.hi - 128u : 0u);
    }
  }

  // Lane offsets of stage k0 (an out-of-range base when the chunk is outside
  // [klo, kend); adding a step to it stays out of range).
  // MASK: a chunk that overlaps [klo, kend) at all is loaded (the bytes outside
  // are zeroed in registers after the fragment reads, mask_frags()).
  __device__ __forceinline__ void stage_base(uint32_t k0, uint32_t& bp, uint32_t& bq) const {
    const uint32_t k = k0 + kcol;
    const bool ok = (MASK ? k + 16u > klo : k >= klo) && k < kend;
    bp = ok ? vp + k0 : kOobOffset;
    bq = ok ? vq + k0 : kOobOffset;
  }

  __device__ __forceinline__ static uint32_t step(uint32_t i, const Operand& X) {
    return ((i >> 2) * X.hi + (i & 3u)) * X.ld;
  }

  __device__ __forceinline__ void load_p(uint8_t* stage, const Operand& P, uint32_t bp,
                                         uint32_t i) const {
    dma_x4(P.data, lds_offset(stage) + 4096u * i + 1024u * wave_id(), bp, step(i, P));
  }
  __device__ __forceinline__ void load_q(uint8_t* stage, const Operand& Q, uint32_t bq,
                                         uint32_t i) const {
    dma_x4(Q.data, lds_offset(stage) + kOpBytes + 4096u * i + 1024u * wave_id(),
           bq, step(i, Q));
  }
  // Scale rows of k-block k0/32 + wave; operand X = P (OP 0) or Q (OP 1).
  template <int OP>
  __device__ __forceinline__ void load_scale(uint8_t* stage, const Operand& X, uint32_t k0) const {
    if (!SCALED) return;
    const uint32_t wave = wave_id();
    const uint32_t blk = (k0 >> 5) + wave;
    const bool ok = blk >= (klo >> 5) && blk < (kend >> 5);
    // the block's row offset is wave-uniform: it rides in the scalar offset,
    // and an out-of-range block moves the whole load past num_records
    dma_x1(X.scale, lds_offset(stage) + kScaleOff + kScaleBlk * wave + 256u * OP, OP ? sq : sp,
           ok ? blk * X.lds : kOobOffset);
  }

  // The 16 data loads of one stage, back to back (prologue only).
  __device__ __forceinline__ void issue_data(uint8_t* stage, const Operand& P, const Operand& Q,
                                             uint32_t k0) const {
    uint32_t bp, bq;
    stage_base(k0, bp, bq);
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) load_p(stage, P, bp, i);
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) load_q(stage, Q, bq, i);
  }
};

// Operands of one stage in registers: 8 P fragments and 8 Q fragments of 16
// rows x 128 contraction bytes, and the scale dwords of the lane's 32-block
// for the P rows of fragment halves G = 0, 1 (sa[G]) and the Q rows of
// halves H = 0, 1 (sb[H]).
struct Frags {
  v8i a[8], b[8];
  uint32_t sa[2], sb[2];
};

// Per-lane LDS byte offsets (relative to a stage).
//   v_mfma_scale_f32_16x16x128_f8f6f4 (fp8) operand layout: lane m + 16g
//   serves row m of a fragment with contraction chunks g (bytes 0..15) and
//   g + 4 (bytes 16..31) of the 128-deep stage, the scale of 32-block b of
//   row m comes from lane m + 16b, and D[4g + r][c] sits in register r of
//   lane c + 16g.  Fragment f = 4G + i of wave row-half w holds tile rows
//   128w + 64G + 4m + i (m = 0..15): LDS slots 128w + 32i + 16G + m of the
//   DMA's slot layout.  Its scale byte is byte i of the dword of rows
//   128w + 64G + 4m .. +3 of the lane's block.
struct FragAddr {
  uint32_t plo, phi, qlo, qhi, ps, qs;

  __device__ __forceinline__ void init() {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t wp = wave & 1u, wq = wave >> 1;
    const uint32_t m = lane & 15u, g = lane >> 4;
    // swz(128w + 32i + 16G + m) = swz(m) for every w, i, G
    const uint32_t sw = swz(m);
    const uint32_t rp = (wp * 128u + m) * kStageK, rq = kOpBytes + (wq * 128u + m) * kStageK;
    plo = rp + ((g ^ sw) << 4);
    phi = rp + (((g + 4u) ^ sw) << 4);
    qlo = rq + ((g ^ sw) << 4);
    qhi = rq + (((g + 4u) ^ sw) << 4);
    ps = kScaleOff + g * kScaleBlk + wp * 128u + 4u * m;
    qs = kScaleOff + 256u + g * kScaleBlk + wq * 128u + 4u * m;
  }
};

// Byte offset of fragment f = 4G + i from fragment 0: 16G + 32i slots.
constexpr uint32_t frag_off(int f) {
  return 2048u * (uint32_t)(f >> 2) + 4096u * (uint32_t)(f & 3);
}

__device__ __forceinline__ v8i lds_v8i(const uint8_t* lo, const uint8_t* hi) {
  const uint4 a = *reinterpret_cast<const uint4*>(lo);
  const uint4 b = *reinterpret_cast<const uint4*>(hi);
  v8i f;
  f[0] = (int)a.x; f[1] = (int)a.y; f[2] = (int)a.z; f[3] = (int)a.w;
  f[4] = (int)b.x; f[5] = (int)b.y; f[6] = (int)b.z; f[7] = (int)b.w;
  return f;
}

template <int F>
__device__ __forceinline__ void read_a(const uint8_t* stage, const FragAddr& fa, Frags& f) {
  f.a[F] = lds_v8i(stage + fa.plo + frag_off(F), stage + fa.phi + frag_off(F));
}
template <int F>
__device__ __forceinline__ void read_b(const uint8_t* stage, const FragAddr& fa, Frags& f) {
  f.b[F] = lds_v8i(stage + fa.qlo + frag_off(F), stage + fa.qhi + frag_off(F));
}
// Unscaled kernels use scale byte 127 (2^0) in every position.
template <bool SCALED, int G>
__device__ __forceinline__ void read_sa(const uint8_t* stage, const FragAddr& fa, Frags& f) {
  f.sa[G] = SCALED ? *reinterpret_cast<const uint32_t*>(stage + fa.ps + 64u * G) : 0x7F7F7F7Fu;
}
template <bool SCALED, int H>
__device__ __forceinline__ void read_sb(const uint8_t* stage, const FragAddr& fa, Frags& f) {
  f.sb[H] = SCALED ? *reinterpret_cast<const uint32_t*>(stage + fa.qs + 64u * H) : 0x7F7F7F7Fu;
}

// One MFMA: P fragment PI against Q fragment QJ into accumulator 8 PI + QJ;
// op_sel picks byte PI % 4 of the P scale dword of half PI / 4 and byte
// QJ % 4 of the Q dword of half QJ / 4.
template <int PI, int QJ>
__device__ __forceinline__ void mma(const Frags& f, v4f (&acc)[64]) {
  acc[8 * PI + QJ] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
      f.a[PI], f.b[QJ], acc[8 * PI + QJ], 0, 0, PI & 3, (int)f.sa[PI >> 2], QJ & 3,
      (int)f.sb[QJ >> 2]);
}

// Bytes of the 4-byte word at contraction position c that lie in [klo, kend),
// as a byte mask (0xFF per byte inside).
__device__ __forceinline__ uint32_t bytes_below(int n) {
  return n <= 0 ? 0u : (n >= 4 ? 0xFFFFFFFFu : (1u << (8 * n)) - 1u);
}
__device__ __forceinline__ uint32_t word_window(uint32_t c, uint32_t klo, uint32_t kend) {
  return bytes_below((int)kend - (int)c) & ~bytes_below((int)klo - (int)c);
}

// Byte masks of the lane's eight fragment dwords for the stage starting at
// k0: dwords 0..3 hold contraction chunk g (bytes k0 + 16g ..), dwords 4..7
// chunk g + 4.  Every fragment of the stage shares them.
struct KMask {
  uint32_t m[8];
};
__device__ __forceinline__ void k_mask(KMask& km, uint32_t k0, uint32_t klo, uint32_t kend) {
  const uint32_t g = (threadIdx.x & 63u) >> 4;
  const uint32_t clo = k0 + 16u * g, chi = clo + 64u;
#pragma unroll
  for (uint32_t d = 0; d < 4; ++d) {
    km.m[d] = word_window(clo + 4u * d, klo, kend);
    km.m[4 + d] = word_window(chi + 4u * d, klo, kend);
  }
}
// Zero the bytes of a fragment outside [klo, kend) (in both operands: a zero on
// one side alone would still turn a NaN code on the other into NaN).
__device__ __forceinline__ void apply_mask(v8i& x, const KMask& km) {
#pragma unroll
  for (int d = 0; d < 8; ++d) x[d] &= (int)km.m[d];
}

#define MXGG_FENCE() __builtin_amdgcn_sched_barrier(0)

// Workgroup barrier after this wave's LDS reads have returned (no wait on
// the DMA), as assembly for the same reason as wait_barrier().
__device__ __forceinline__ void release_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Accumulate D over k in [klo, kend) (both multiples of 32).  The stages start
// at klo rounded down to 128 so that every stage reads whole cache lines of
// rows whose stride is a multiple of 128; chunks below klo load as zeros.
//
// Stage s lives in slot s%2.  Its 64 MFMAs run P fragments 0..7 against Q
// fragments 0..3 (MFMA n = 4p + q), then against Q fragments 4..7 (n = 32 +
// 4p + q - 4).  Fragment registers are refilled as they free up, so one set of
// 128 VGPRs holds two stages at once and every read has MFMAs to land in:
//     0-8  the rest of stage s from slot s%2: P 4..7 (first used at 16..28),
//          the P scales of half 1 (first used at 16), Q 4..7 and the Q
//          scales of half 1 (first used at 32)
//      12  release barrier: every wave has read all of slot s%2 -> the 18
//          loads of stage s+2 into that slot, one per about three MFMAs up to
//          MFMA 62
//      32  publish barrier: everything older than the 7 loads issued since
//          the release, i.e. all of stage s+1, has landed
//   33-58  the first part of stage s+1 from the other slot: Q 0..3 (free since
//          MFMA 31) and P 0..3, each after its last use in stage s (MFMA
//          35 + 4p), and the scales of halves 0
// A load has at least 34 MFMAs (about 1100 cycles) to land before its
// publish.  Releasing later (MFMA 16 to 24) or placing the loads and reads on
// MFMA pairs measured slower.  The wait counts do not depend on whether
// scales are loaded: the scale loads of a stage come after its data loads,
// and the publish wait leaves exactly the 7 newest (data) loads in flight.
// MASK (unscaled only): [klo, kend) may have any bounds; chunks that straddle
// them are loaded whole and the bytes outside are zeroed in registers right
// after each fragment read.  Only experts whose token range is not a multiple
// of 16 take this path.
template <bool SCALED, bool MASK = false>
__device__ __forceinline__ void mainloop(Smem& sm, const Operand& P, const Operand& Q,
                                         uint32_t klo, uint32_t kend, v4f (&acc)[64]) {
  static_assert(!(SCALED && MASK), "a scale block cannot be split by a token mask");
#pragma unroll
  for (int i = 0; i < 64; ++i) acc[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  if (kend <= klo) return;
  const uint32_t kbeg = klo & ~(uint32_t)(kStageK - 1);
  const uint32_t nst = (kend - kbeg + kStageK - 1) / kStageK;
  Stream<SCALED, MASK> st;
  st.init(P, Q, klo, kend);
  FragAddr fa;
  fa.init();
  // Prologue: all of stage 0 and the data of stage 1 (its scales follow in
  // the first stage), then publish stage 0 and read the part of it that the
  // loop reads one stage ahead.
  st.template load_scale<0>(sm.ring[0], P, kbeg);
  st.template load_scale<1>(sm.ring[0], Q, kbeg);
  st.issue_data(sm.ring[0], P, Q, kbeg);
  st.issue_data(sm.ring[1], P, Q, kbeg + kStageK);
  st.template load_scale<0>(sm.ring[1], P, kbeg + kStageK);
  st.template load_scale<1>(sm.ring[1], Q, kbeg + kStageK);
  wait_barrier<SCALED ? 18 : 16>();
  MXGG_FENCE();
  Frags f;
  KMask km;
  if constexpr (MASK) k_mask(km, kbeg, klo, kend);
#define MASKA(F) \
  if constexpr (MASK) apply_mask(f.a[F], km)
#define MASKB(F) \
  if constexpr (MASK) apply_mask(f.b[F], km)
  {
    const uint8_t* r0 = sm.ring[0];
    read_b<0>(r0, fa, f); MASKB(0);
    read_b<1>(r0, fa, f); MASKB(1);
    read_b<2>(r0, fa, f); MASKB(2);
    read_b<3>(r0, fa, f); MASKB(3);
    read_a<0>(r0, fa, f); MASKA(0);
    read_a<1>(r0, fa, f); MASKA(1);
    read_a<2>(r0, fa, f); MASKA(2);
    read_a<3>(r0, fa, f); MASKA(3);
    read_sa<SCALED, 0>(r0, fa, f);
    read_sb<SCALED, 0>(r0, fa, f);
  }
  // Past the last stage the loads fetch zeros into a slot nobody reads again,
  // and the final reads fetch a stale slot that is never used, so the loop
  // body has no branches.  nst >= 1 here (kend > klo); written as a do-while
  // because a loop that may run zero times made the compiler zero the
  // accumulators twice per tile, once for the zero-trip path.
  uint32_t s = 0;
  do {
    uint8_t* cur = sm.ring[s & 1u];
    uint8_t* nxt = sm.ring[(s & 1u) ^ 1u];
    uint32_t bp, bq;
    st.stage_base(kbeg + (s + 2) * kStageK, bp, bq);
      mma<0, 0>(f, acc); read_a<4>(cur, fa, f); MASKA(4); MXGG_FENCE();
      mma<0, 1>(f, acc); read_sa<SCALED, 1>(cur, fa, f); MXGG_FENCE();
      mma<0, 2>(f, acc); read_a<5>(cur, fa, f); MASKA(5); MXGG_FENCE();
      mma<0, 3>(f, acc); read_b<4>(cur, fa, f); MASKB(4); MXGG_FENCE();
      mma<1, 0>(f, acc); read_a<6>(cur, fa, f); MASKA(6); MXGG_FENCE();
      mma<1, 1>(f, acc); read_b<5>(cur, fa, f); MASKB(5); MXGG_FENCE();
      mma<1, 2>(f, acc); read_a<7>(cur, fa, f); MASKA(7); MXGG_FENCE();
      mma<1, 3>(f, acc); read_b<6>(cur, fa, f); MASKB(6); MXGG_FENCE();
      mma<2, 0>(f, acc); read_sb<SCALED, 1>(cur, fa, f); read_b<7>(cur, fa, f); MASKB(7); MXGG_FENCE();
      mma<2, 1>(f, acc); MXGG_FENCE();
      mma<2, 2>(f, acc); MXGG_FENCE();
      mma<2, 3>(f, acc); MXGG_FENCE();
      release_barrier();
      MXGG_FENCE();
      mma<3, 0>(f, acc); st.load_p(cur, P, bp, 0); MXGG_FENCE();
      mma<3, 1>(f, acc); MXGG_FENCE();
      mma<3, 2>(f, acc); MXGG_FENCE();
      mma<3, 3>(f, acc); st.load_p(cur, P, bp, 1); MXGG_FENCE();
      mma<4, 0>(f, acc); MXGG_FENCE();
      mma<4, 1>(f, acc); MXGG_FENCE();
      mma<4, 2>(f, acc); st.load_p(cur, P, bp, 2); MXGG_FENCE();
      mma<4, 3>(f, acc); MXGG_FENCE();
      mma<5, 0>(f, acc); MXGG_FENCE();
      mma<5, 1>(f, acc); st.load_p(cur, P, bp, 3); MXGG_FENCE();
      mma<5, 2>(f, acc); MXGG_FENCE();
      mma<5, 3>(f, acc); MXGG_FENCE();
      mma<6, 0>(f, acc); st.load_p(cur, P, bp, 4); MXGG_FENCE();
      mma<6, 1>(f, acc); MXGG_FENCE();
      mma<6, 2>(f, acc); MXGG_FENCE();
      mma<6, 3>(f, acc); st.load_p(cur, P, bp, 5); MXGG_FENCE();
      mma<7, 0>(f, acc); MXGG_FENCE();
      mma<7, 1>(f, acc); MXGG_FENCE();
      mma<7, 2>(f, acc); st.load_p(cur, P, bp, 6); MXGG_FENCE();
      mma<7, 3>(f, acc); MXGG_FENCE();
      wait_barrier<7>();
      MXGG_FENCE();
      if constexpr (MASK) k_mask(km, kbeg + (s + 1) * kStageK, klo, kend);
      mma<0, 4>(f, acc); MXGG_FENCE();
      mma<0, 5>(f, acc); read_b<0>(nxt, fa, f); MASKB(0); MXGG_FENCE();
      mma<0, 6>(f, acc); st.load_p(cur, P, bp, 7); MXGG_FENCE();
      mma<0, 7>(f, acc); MXGG_FENCE();
      mma<1, 4>(f, acc); read_a<0>(nxt, fa, f); MASKA(0); MXGG_FENCE();
      mma<1, 5>(f, acc); st.load_q(cur, Q, bq, 0); MXGG_FENCE();
      mma<1, 6>(f, acc); MXGG_FENCE();
      mma<1, 7>(f, acc); read_b<1>(nxt, fa, f); MASKB(1); MXGG_FENCE();
      mma<2, 4>(f, acc); st.load_q(cur, Q, bq, 1); MXGG_FENCE();
      mma<2, 5>(f, acc); read_a<1>(nxt, fa, f); MASKA(1); MXGG_FENCE();
      mma<2, 6>(f, acc); MXGG_FENCE();
      mma<2, 7>(f, acc); st.load_q(cur, Q, bq, 2); MXGG_FENCE();
      mma<3, 4>(f, acc); MXGG_FENCE();
      mma<3, 5>(f, acc); read_b<2>(nxt, fa, f); MASKB(2); st.load_q(cur, Q, bq, 3); MXGG_FENCE();
      mma<3, 6>(f, acc); read_a<2>(nxt, fa, f); MASKA(2); MXGG_FENCE();
      mma<3, 7>(f, acc); MXGG_FENCE();
      mma<4, 4>(f, acc); st.load_q(cur, Q, bq, 4); MXGG_FENCE();
      mma<4, 5>(f, acc); MXGG_FENCE();
      mma<4, 6>(f, acc); read_a<3>(nxt, fa, f); MASKA(3); MXGG_FENCE();
      mma<4, 7>(f, acc); st.load_q(cur, Q, bq, 5); MXGG_FENCE();
      mma<5, 4>(f, acc); read_b<3>(nxt, fa, f); MASKB(3); MXGG_FENCE();
      mma<5, 5>(f, acc); MXGG_FENCE();
      mma<5, 6>(f, acc); st.load_q(cur, Q, bq, 6); MXGG_FENCE();
      mma<5, 7>(f, acc); read_sb<SCALED, 0>(nxt, fa, f); MXGG_FENCE();
      mma<6, 4>(f, acc); st.load_q(cur, Q, bq, 7); MXGG_FENCE();
      mma<6, 5>(f, acc); MXGG_FENCE();
      mma<6, 6>(f, acc); read_sa<SCALED, 0>(nxt, fa, f); MXGG_FENCE();
      mma<6, 7>(f, acc); st.template load_scale<0>(cur, P, kbeg + (s + 2) * kStageK); MXGG_FENCE();
      mma<7, 4>(f, acc); MXGG_FENCE();
      mma<7, 5>(f, acc); MXGG_FENCE();
      mma<7, 6>(f, acc); st.template load_scale<1>(cur, Q, kbeg + (s + 2) * kStageK); MXGG_FENCE();
      mma<7, 7>(f, acc); MXGG_FENCE();
  } while (++s < nst);
#undef MASKA
#undef MASKB
  // Drain the loads past the end before the next tile's prologue reuses the slots.
  wait_barrier<0>();
}

#undef MXGG_FENCE

// Value of the neighbouring lane (lane ^ 1) through a DPP quad permutation
// [1, 0, 3, 2]: a VALU move, no LDS round trip (unlike a shuffle).
__device__ __forceinline__ uint32_t swap_lane_pair(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false);
}

// Write the tile: output row = Q index in [qbeg, qend), column = P index < pend.
// Register r of accumulator 8(4G + i) + 4H + j in lane c + 16g is D[4g + r][c]
// of the 16x16 MFMA of P fragment 4G + i and Q fragment 4H + j, i.e. P index
// 128wp + 64G + 16g + 4r + i and Q index 128wq + 64H + 4c + j: the four
// fragments i = 0..3 hold one 4-value chunk of consecutive P indices.
// Stored directly, every store instruction would scatter 64 small pieces over
// 16 rows.  Instead each wave stages its 128x128 fp32 sub-tile in its own
// 32 KB of the idle LDS ring, in two passes of 64 rows (j = 0,1 then j = 2,3;
// staged row s = 2(16H + c) + j%2, 512 B), and then stores whole rows: 32
// lanes x 4 values, converted to bf16 after the read for bf16 output.  The 16-byte
// chunk k of staged row s sits at k ^ ((s/2) mod 16), so a half-wave writing
// one chunk column of 32 rows, and one reading a whole row, touches each LDS
// bank exactly twice.  The staging writes take the accumulators straight from
// AGPRs.  The output is written once and not read again by the kernel, so the
// row stores are nontemporal (measured faster, most for fp32 output).
template <bool F32>
__device__ __forceinline__ void epilogue(Smem& sm, const v4f (&acc)[64], char* out,
                                         int64_t ldo_bytes, uint32_t q0, uint32_t qbeg,
                                         uint32_t qend, uint32_t p0, uint32_t pend,
                                         bool accumulate = false) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = wave_id();
  const uint32_t wp = wave & 1u, wq = wave >> 1;
  const uint32_t l32 = lane & 31u, h = lane >> 5;
  const uint32_t c16 = lane & 15u, g = lane >> 4;
  uint8_t* stage = &sm.ring[0][0] + wave * 32768u;
  const uint32_t p = p0 + wp * 128u + 4u * l32;  // this lane's 4 columns on the way out
  // fp32 stores of a wave whose 128 rows and 128 columns all lie inside the
  // output go through one buffer descriptor based at its first row and
  // column: a per-lane offset fixed for the tile plus a scalar row offset per
  // store, no guards.
  const uint32_t qw = q0 + 128u * wq, pw = p0 + 128u * wp;
  const bool interior = F32 && !accumulate && qw >= qbeg && qw + 128u <= qend &&
                        pw + 128u <= pend &&
                        ((reinterpret_cast<uintptr_t>(out) | (uintptr_t)ldo_bytes) & 15u) == 0 &&
                        ldo_bytes < (int64_t)1 << 24;
  const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
      out + (int64_t)qw * ldo_bytes + 4 * (int64_t)pw, (short)0,
      (int)(128u * (uint32_t)ldo_bytes), 0x00020000);
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int qj = 4 * hh + 2 * pass + jj;
        uint8_t* row = stage + (2u * (16u * (uint32_t)hh + c16) + (uint32_t)jj) * 512u;
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t c = 16u * (uint32_t)gg + 4u * g + (uint32_t)r;
            *reinterpret_cast<float4*>(row + ((c ^ c16) << 4)) =
                make_float4(acc[8 * (4 * gg) + qj][r], acc[8 * (4 * gg + 1) + qj][r],
                            acc[8 * (4 * gg + 2) + qj][r], acc[8 * (4 * gg + 3) + qj][r]);
          }
      }
    // This wave's LDS writes complete before its reads (in-order LDS queue).
    // Reads go out eight at a time, unconditionally (they are always in
    // bounds), so their latency overlaps; only the global stores of a
    // boundary wave are guarded.
#pragma unroll
    for (uint32_t t0 = 0; t0 < 32u; t0 += 8u) {
      v4f v[8];
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t t = t0 + u;
        v[u] = *reinterpret_cast<const v4f*>(stage + (2u * t + h) * 512u +
                                             ((l32 ^ (t & 15u)) << 4));
      }
      // keep the reads here instead of letting them sink into the guarded stores
      asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]));
      if constexpr (F32) {
        if (interior) {
          // row 2*pass + h of each group of four, 16 bytes per lane
          const uint32_t voff = (2u * (uint32_t)pass + h) * (uint32_t)ldo_bytes + 16u * l32;
#pragma unroll
          for (uint32_t u = 0; u < 8u; ++u)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[u]), rows, voff,
                                                   4u * (t0 + u) * (uint32_t)ldo_bytes, kCacheNT);
          continue;
        }
#pragma unroll
        for (uint32_t u = 0; u < 8u; ++u) {
          const uint32_t q = q0 + wq * 128u + 4u * (t0 + u) + 2u * (uint32_t)pass + h;
          if (q < qbeg || q >= qend || p >= pend) continue;
          float* dst = reinterpret_cast<float*>(out + (int64_t)q * ldo_bytes) + p;
          if (accumulate) {
            // split-K partial sum: vector fp32 atomics into the zeroed output
            for (uint32_t k = 0; k < 4u && p + k < pend; ++k)
              __hip_atomic_fetch_add(dst + k, v[u][k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else if (p + 4u <= pend) {
            __builtin_nontemporal_store(v[u], reinterpret_cast<v4f*>(dst));
          } else {
            for (uint32_t k = 0; p + k < pend; ++k) dst[k] = v[u][k];
          }
        }
      } else {
        // bf16: 8 bytes per lane and row.  Lanes 2i and 2i+1 swap halves of two
        // consecutive rows so that each holds 8 consecutive values of one row
        // and stores 16 bytes: the even lane row t at columns p..p+7, the odd
        // lane row t+1 at p-4..p+3.
        const bool odd = (l32 & 1u) != 0;
        const uint32_t pe = p0 + wp * 128u + 8u * (l32 >> 1);
#pragma unroll
        for (uint32_t u = 0; u < 8u; u += 2u) {
          const uint2 a = make_uint2(pack_bf16x2(v[u][0], v[u][1]), pack_bf16x2(v[u][2], v[u][3]));
          const uint2 b =
              make_uint2(pack_bf16x2(v[u + 1][0], v[u + 1][1]), pack_bf16x2(v[u + 1][2], v[u + 1][3]));
          const uint2 send = odd ? a : b;
          const uint2 recv = make_uint2(swap_lane_pair(send.x), swap_lane_pair(send.y));
          const uint4 row8 = odd ? make_uint4(recv.x, recv.y, b.x, b.y)
                                 : make_uint4(a.x, a.y, recv.x, recv.y);
          const uint32_t t = t0 + u + (odd ? 1u : 0u);
          const uint32_t q = q0 + wq * 128u + 4u * t + 2u * (uint32_t)pass + h;
          if (q < qbeg || q >= qend || pe >= pend) continue;
          uint16_t* dst = reinterpret_cast<uint16_t*>(out + (int64_t)q * ldo_bytes) + pe;
          if (pe + 8u <= pend && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
            __builtin_nontemporal_store(u32x4{row8.x, row8.y, row8.z, row8.w}, reinterpret_cast<u32x4*>(dst));
          } else {
            const uint32_t w[4] = {row8.x, row8.y, row8.z, row8.w};
            for (uint32_t k = 0; k < 8u && pe + k < pend; ++k)
              dst[k] = (uint16_t)(w[k >> 1] >> (16u * (k & 1u)));
          }
        }
      }
    }
  }
  // Every wave has read its staging area before the next tile's loads land in the ring.
  __syncthreads();
}

// Epilogue of the fused gate+up forward: the tile's P rows are 128 gate rows
// (waves wp = 0) and the 128 matching up rows (wp = 1), so a = SiLU(gate) * up
// of 128 consecutive features of 256 tokens is formed here and written as its
// row-wise MXFP8 cast: e4m3 payload aq[token][pg + f] and one E8M0 byte per
// 32 features at s[token * s_row + block * s_blk].  The bf16 gate+up output h
// of the unfused path never reaches HBM (33 KB written per tile instead of
// 128 KB).  The arithmetic is the unfused path's: h rounded to bf16, then
// swiglu_a_chunk and the dim0 cast rule of the standalone kernels.
//   1. every wave stages its 128 x 128 sub-tile as bf16 in the idle LDS ring:
//      row q (token) x 512 B, gate columns in 16-byte chunks 0..15, up in
//      16..31, chunk index XOR-swizzled by (q / 4) mod 16 (each half-wave then
//      touches every bank at most twice, writing and reading);
//   2. lane (qq, k) of wave w takes token 64w + 4i + qq and features
//      8k .. 8k+7 on trip i: one 16-byte read of gate and of up, SwiGLU,
//      block amax over the quad k = 4b .. 4b+3, 8 payload bytes (16 lanes
//      write one 128-byte row piece), the quad's first lane the scale byte.
// The tile rounded to bf16 and staged in the idle LDS ring as 256 rows (Q
// index) x 512 B (P index 0..255), 16-byte chunk k of row q at chunk
// k ^ ((q / 4) mod 16): a half-wave writing one chunk column of 32 rows, or
// reading one whole row, touches every bank at most twice.
__device__ __forceinline__ void stage_bf16_tile(Smem& sm, const v4f (&acc)[64]) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t wp = wave & 1u, wq = wave >> 1;
  const uint32_t c16 = lane & 15u, g = lane >> 4;
  uint8_t* st = &sm.ring[0][0];
#pragma unroll
  for (uint32_t qj = 0; qj < 8; ++qj) {
    // Q row 128wq + 64H + 4c + j of fragment qj = 4H + j; its swizzle
    // ((row / 4) mod 16) is c
    const uint32_t q = 128u * wq + 64u * (qj >> 2) + 4u * c16 + (qj & 3u);
    uint8_t* row = st + q * 512u;
#pragma unroll
    for (uint32_t gg = 0; gg < 2; ++gg)
#pragma unroll
      for (uint32_t b = 0; b < 2; ++b) {
        // registers 2b and 2b + 1 of P fragments 4gg .. 4gg+3 hold P columns
        // 64gg + 16g + 8b .. +7 of the wave's half
        const uint32_t r = 2u * b;
        const uint32_t chunk = 16u * wp + 8u * gg + 2u * g + b;
        const uint32_t a0 = 8u * (4u * gg) + qj;
        *reinterpret_cast<uint4*>(row + ((chunk ^ c16) << 4)) =
            make_uint4(pack_bf16x2(acc[a0][r], acc[a0 + 8u][r]),
                       pack_bf16x2(acc[a0 + 16u][r], acc[a0 + 24u][r]),
                       pack_bf16x2(acc[a0][r + 1u], acc[a0 + 8u][r + 1u]),
                       pack_bf16x2(acc[a0 + 16u][r + 1u], acc[a0 + 24u][r + 1u]));
      }
  }
  __syncthreads();
}

// bf16 output through the bf16 staging: wave w stores rows 64w .. 64w+63 of
// the tile, two whole 512-byte rows per store instruction (lanes 0-31 one
// row, 32-63 the next).
__device__ __forceinline__ void epilogue_bf16(Smem& sm, const v4f (&acc)[64], char* out,
                                              int64_t ldo_bytes, uint32_t q0, uint32_t qbeg,
                                              uint32_t qend, uint32_t p0, uint32_t pend) {
  stage_bf16_tile(sm, acc);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = wave_id();
  const uint32_t c = lane & 31u;
  const uint32_t p = p0 + 8u * c;
  const uint8_t* st = &sm.ring[0][0];
  // A wave whose 64 rows and 256 columns all lie inside the output stores
  // through one buffer descriptor based at its first row: a per-lane offset
  // fixed for the tile plus a scalar row offset per store, no guards.
  const uint32_t qw = q0 + 64u * wave;
  const bool interior = qw >= qbeg && qw + 64u <= qend && p0 + 256u <= pend &&
                        ((reinterpret_cast<uintptr_t>(out) | (uintptr_t)ldo_bytes) & 15u) == 0 &&
                        ldo_bytes < (int64_t)1 << 25;
  const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
      out + (int64_t)qw * ldo_bytes + 2 * (int64_t)p0, (short)0,
      (int)(64u * (uint32_t)ldo_bytes), 0x00020000);
  const uint32_t voff = (lane >> 5) * (uint32_t)ldo_bytes + 16u * c;
#pragma unroll
  for (uint32_t i0 = 0; i0 < 32u; i0 += 8u) {
    u32x4 v[8];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t q = 64u * wave + 2u * (i0 + u) + (lane >> 5);
      v[u] = *reinterpret_cast<const u32x4*>(st + q * 512u + ((c ^ ((q >> 2) & 15u)) << 4));
    }
    // keep the reads here instead of letting them sink into the guarded stores
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                 "+v"(v[6]), "+v"(v[7]));
    if (interior) {
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u)
        __builtin_amdgcn_raw_buffer_store_b128(v[u], rows, voff,
                                               2u * (i0 + u) * (uint32_t)ldo_bytes, kCacheNT);
      continue;
    }
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
      const uint32_t q = q0 + 64u * wave + 2u * (i0 + u) + (lane >> 5);
      if (q < qbeg || q >= qend || p >= pend) continue;
      uint16_t* dst = reinterpret_cast<uint16_t*>(out + (int64_t)q * ldo_bytes) + p;
      if (p + 8u <= pend && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        __builtin_nontemporal_store(v[u], reinterpret_cast<u32x4*>(dst));
      } else {
        for (uint32_t k = 0; k < 8u && p + k < pend; ++k)
          dst[k] = (uint16_t)(v[u][k >> 1] >> (16u * (k & 1u)));
      }
    }
  }
  // every wave has read the staging area before the next tile's loads land
  __syncthreads();
}

// KEEP: the bf16 gate and up values are also stored, as h[tok][pg + c] and
// h[tok][F + pg + c] (ldh elements per row), for a backward that re-reads h:
// the same bits epilogue_bf16 writes for the unfused projection.
template <int MODE, bool KEEP>
__device__ __forceinline__ void epilogue_swiglu(Smem& sm, const v4f (&acc)[64], uint8_t* aq,
                                                int64_t ldq, uint8_t* sc, int64_t s_row,
                                                int64_t s_blk, uint32_t q0, uint32_t qbeg,
                                                uint32_t qend, uint32_t pg, uint16_t* h,
                                                int64_t ldh, uint32_t F) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  uint8_t* st = &sm.ring[0][0];
  stage_bf16_tile(sm, acc);
  const uint32_t k = lane & 15u, qq = lane >> 4;
#pragma unroll 2
  for (uint32_t i = 0; i < 16u; ++i) {
    const uint32_t q = 64u * wave + 4u * i + qq;
    const uint32_t sw = (q >> 2) & 15u;
    const uint8_t* row = st + q * 512u;
    const uint4 g = *reinterpret_cast<const uint4*>(row + ((k ^ sw) << 4));
    const uint4 u = *reinterpret_cast<const uint4*>(row + ((16u + (k ^ sw)) << 4));
    const uint32_t tok = q0 + q;
    // h first: its stores drain while the activation is computed
    if (KEEP && tok >= qbeg && tok < qend) {
      uint16_t* hr = h + (int64_t)tok * ldh + pg + 8u * k;
      __builtin_nontemporal_store(u32x4{g.x, g.y, g.z, g.w}, reinterpret_cast<u32x4*>(hr));
      __builtin_nontemporal_store(u32x4{u.x, u.y, u.z, u.w}, reinterpret_cast<u32x4*>(hr + F));
    }
    const uint4 a = swiglu_a_chunk(g, u);
    uint32_t am = amax16_of_chunk(a);
    am = quad_max(am);
    const uint32_t b = e8m0_from_amax16<MODE>(am);
    const uint2 o = __any(needs_full_encoder<MODE, false>(b))
                        ? encode_chunk8<MODE, false, true>(a, b)
                        : encode_chunk8<MODE, false, false>(a, b);
    if (tok >= qbeg && tok < qend) {
      *reinterpret_cast<uint2*>(aq + (int64_t)tok * ldq + pg + 8u * k) = o;
      if ((k & 3u) == 0)
        sc[(int64_t)tok * s_row + (int64_t)((pg >> 5) + (k >> 2)) * s_blk] = (uint8_t)b;
    }
  }
  // every wave has read the staging area before the next tile's loads land
  __syncthreads();
}

// Decode a position in the tile order into (mt, nt): bands of `gm`
// consecutive m-tiles are walked column by column so that neighbouring tiles
// share either their Q rows or their P rows.
__device__ __forceinline__ void band_decode(uint32_t lid, uint32_t m_tiles, uint32_t n_tiles,
                                            uint32_t gm, uint32_t& mt, uint32_t& nt) {
  const uint32_t per_band = gm * n_tiles;
  const uint32_t band = lid / per_band;
  const uint32_t first = band * gm;
  const uint32_t width = min(gm, m_tiles - first);
  const uint32_t in = lid - band * per_band;
  nt = in / width;
  mt = first + (in - nt * width);
}

// Largest index i < n with a[i] <= v in a non-decreasing LDS array (a[0] <= v),
// found by the whole wave at once: one LDS read and a ballot per 64 entries
// instead of a chain of dependent reads.
__device__ __forceinline__ int last_le(const int32_t* a, int n, uint32_t v) {
  const int lane = (int)(threadIdx.x & 63u);
  int best = 0;
  for (int base = 0; base < n; base += 64) {
    const int i = base + lane;
    const uint64_t m = __ballot(i < n && (uint32_t)a[i] <= v);
    if (m != 0) best = base + 63 - __clzll((long long)m);
    if (m != ~0ull) break;
  }
  return best;
}

// Position in the global tile order processed by this workgroup at round
// `base`: each XCD (workgroups are dealt to the 8 XCDs round-robin) takes a
// contiguous slice of the round.
__device__ __forceinline__ uint32_t xcd_slice(uint32_t base) {
  const uint32_t g = gridDim.x;  // multiple of 8
  return base + (blockIdx.x & 7u) * (g >> 3) + (blockIdx.x >> 3);
}

// Block-wide inclusive scan of per-group counts into out[1..E] (out[0] = 0),
// both arrays in LDS.  Each thread owns 4 consecutive groups.
__device__ void scan_counts(Smem& sm, const int32_t* tiles_of, int32_t* out, int E) {
  const int t = threadIdx.x;
  int32_t loc[4];
  int32_t sum = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int g = 4 * t + u;
    loc[u] = g < E ? tiles_of[g] : 0;
    sum += loc[u];
  }
  sm.scan_tmp[t] = sum;
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {
    const int32_t add = t >= off ? sm.scan_tmp[t - off] : 0;
    __syncthreads();
    sm.scan_tmp[t] += add;
    __syncthreads();
  }
  int32_t run = t > 0 ? sm.scan_tmp[t - 1] : 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int g = 4 * t + u;
    run += loc[u];
    if (g < E) out[g + 1] = run;
  }
  if (t == 0) out[0] = 0;
  __syncthreads();
}

// Rows [beg, end) of group g from the monotone group ends staged in LDS.
__device__ __forceinline__ void group_range(const int32_t* gend, int g, int32_t& beg,
                                            int32_t& end) {
  beg = g > 0 ? gend[g - 1] : 0;
  end = gend[g];
}

// ---------------------------------------------------------------------------
// Forward: out[m][n] = sum_k A[m][k] W[g][n][k] for m in group g.  The m-tiles
// of a group start at the group's first row rounded down to a multiple of 4
// (the scale DMA copies 4 rows per lane); rows outside the group are computed
// but not stored.
// ---------------------------------------------------------------------------
// Output of the forward: bf16 or fp32 out[m][n], or (SWIGLU_*) the MXFP8
// cast of SiLU(gate) * up for a weight holding [gate; up] rows, with
// (SWIGLU_KEEP_*) or without the bf16 [gate | up] rows in `out`.
enum {
  kOutBf16 = 0,
  kOutF32 = 1,
  kOutSwigluRceil = 2,
  kOutSwigluFloor = 3,
  kOutSwigluKeepRceil = 4,
  kOutSwigluKeepFloor = 5
};

template <bool SCALED, int OUT>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_fwd(FwdArgs args, uint32_t gm) {
  constexpr bool F32 = OUT == kOutF32;
  constexpr bool SWIGLU = OUT >= kOutSwigluRceil;
  constexpr bool KEEP = OUT >= kOutSwigluKeepRceil;
  constexpr int SW_MODE =
      (OUT == kOutSwigluRceil || OUT == kOutSwigluKeepRceil) ? kModeRceil : kModeFloor;
  __shared__ Smem sm;
  const int E = args.group_ends ? args.E : 1;
  const int32_t M = args.M;
  if (args.group_ends)
    monotone_ends_to_lds(args.group_ends, E, M, sm.gend);
  else if (threadIdx.x == 0)
    sm.gend[0] = M;
  __syncthreads();
  for (int g = threadIdx.x; g < E; g += kThreads) {
    int32_t b, e;
    group_range(sm.gend, g, b, e);
    sm.order[g] = e > b ? (e - (b & ~3) + kTileQ - 1) / kTileQ : 0;
  }
  __syncthreads();
  scan_counts(sm, sm.order, sm.sched, E);
  const uint32_t m_tiles = (uint32_t)sm.sched[E];
  // SWIGLU: N = 2F weight rows; a tile covers 128 features of a (F % 128 == 0)
  const uint32_t n_tiles = SWIGLU ? (uint32_t)args.N / 256u
                                  : ((uint32_t)args.N + kTileP - 1) / kTileP;
  const uint32_t total = m_tiles * n_tiles;
  const uint32_t K = (uint32_t)args.K;
  // With a workspace, a last round of tiles that would leave at least half of
  // the workgroups idle is cut along K into S ranges (whole stages), one work
  // item each; k_fwd_split_reduce adds the S partials in a fixed order.
  const uint32_t G = gridDim.x;
  const uint32_t full = total / G * G;
  const uint32_t rem = total - full;
  const uint32_t nst = (K + kStageK - 1) / kStageK;
  uint32_t S = 1, chunk = nst;
  if (args.split_ws != nullptr && rem > 0 && rem <= G / 2 && nst > 1) {
    S = min(min(G / rem, nst), full > 0 ? kMaxSplitTail : kMaxSplit);
    chunk = (nst + S - 1) / S;
    S = (nst + chunk - 1) / chunk;
  }
  int32_t* hdr = reinterpret_cast<int32_t*>(args.split_ws);
  if (hdr != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    hdr[0] = S > 1 ? (int32_t)rem : 0;
    hdr[1] = (int32_t)S;
  }
  const uint32_t items = S > 1 ? full + rem * S : total;

  for (uint32_t base = 0;; base += G) {
    const uint32_t lid = xcd_slice(base);
    if (lid >= items) break;
    uint32_t tile = lid, split = 0;
    const bool part = S > 1 && lid >= full;
    if (part) {
      tile = full + (lid - full) / S;
      split = (lid - full) % S;
    }
    uint32_t mt, nt;
    band_decode(tile, m_tiles, n_tiles, gm, mt, nt);
    // group of m-tile mt: last g with sched[g] <= mt
    const int g = last_le(sm.sched, E, mt);
    int32_t gb, ge;
    group_range(sm.gend, g, gb, ge);
    const uint32_t q0 = (uint32_t)(gb & ~3) + (mt - (uint32_t)sm.sched[g]) * kTileQ;
    const uint32_t p0 = nt * (SWIGLU ? 128u : kTileP);

    Operand P, Q;
    const uint8_t* wg = args.w + (int64_t)g * args.w_gstride;
    P.data = make_desc(wg, (uint32_t)((int64_t)(args.N - 1) * args.ldw + K));
    P.ld = (uint32_t)args.ldw;
    P.row0 = p0;
    P.hi = SWIGLU ? (uint32_t)args.N / 2u : 128u;
    // The A range ends at the group's last row (ge >= 1: empty groups have no
    // tiles), so the rows of a partial m-tile past the group end load as zeros
    // instead of the next expert's rows: no fetch, and the matrix cores run
    // on zeros there (C2 +2%, C3 +1%; those rows are never stored).
    Q.data = make_desc(args.a, (uint32_t)((int64_t)(__builtin_amdgcn_readfirstlane(ge) - 1) *
                                              args.lda + K));
    Q.ld = (uint32_t)args.lda;
    Q.row0 = q0;
    Q.hi = 128u;
    if (SCALED) {
      const uint8_t* wsg = args.ws + (int64_t)g * args.ws_gstride;
      P.scale = make_desc(wsg, scale_extent(K / 32, args.ldws, args.N));
      P.lds = (uint32_t)args.ldws;
      Q.scale = make_desc(args.as, scale_extent(K / 32, args.ldas, M));
      Q.lds = (uint32_t)args.ldas;
    }
    v4f acc[64];
    if (part) {
      const uint32_t klo = split * chunk * kStageK;
      mainloop<SCALED>(sm, P, Q, klo, min(K, klo + chunk * kStageK), acc);
      const uint32_t t = tile - full;
      if (split == 0 && threadIdx.x == 0) {
        hdr[4 + 4 * t] = (int32_t)q0;
        hdr[5 + 4 * t] = (int32_t)p0;
        hdr[6 + 4 * t] = gb;
        hdr[7 + 4 * t] = ge;
      }
      // the whole 256x256 fp32 partial, rows and columns unmasked
      char* slot = reinterpret_cast<char*>(args.split_ws) + kSplitHdrBytes +
                   (int64_t)(t * S + split) * kPartialBytes;
      epilogue<true>(sm, acc, slot, 1024, 0u, 0u, 256u, 0u, 256u);
    } else if constexpr (SWIGLU) {
      mainloop<SCALED>(sm, P, Q, 0u, K, acc);
      epilogue_swiglu<SW_MODE, KEEP>(sm, acc, args.aq, args.ldaq, args.as_out, args.as_row,
                                     args.as_blk, q0, (uint32_t)gb, (uint32_t)ge, p0,
                                     static_cast<uint16_t*>(args.out), args.ldo,
                                     (uint32_t)args.N / 2u);
    } else {
      mainloop<SCALED>(sm, P, Q, 0u, K, acc);
      const int64_t ldo_bytes = args.ldo * (F32 ? 4 : 2);
      if constexpr (F32)
        epilogue<true>(sm, acc, reinterpret_cast<char*>(args.out), ldo_bytes, q0, (uint32_t)gb,
                       (uint32_t)ge, p0, (uint32_t)args.N);
      else
        epilogue_bf16(sm, acc, reinterpret_cast<char*>(args.out), ldo_bytes, q0, (uint32_t)gb,
                      (uint32_t)ge, p0, (uint32_t)args.N);
    }
  }
}

// Sum of the split partials of the forward's last round, in split order (the
// first partial is the starting value), stored inside the tile's group and
// columns.  Each thread takes 4 (tile, row, 4-column) items a grid-stride
// apart and issues all their loads before adding, so the sums are bound by
// bandwidth, not by one load latency per partial.  Exits at once when the
// forward did not split (header count 0).
constexpr int kReduceItems = 4;

__global__ __launch_bounds__(256) void k_fwd_split_reduce(const float* __restrict__ ws,
                                                          void* __restrict__ out, int64_t ldo,
                                                          int32_t N, int32_t out_f32) {
  const int32_t* hdr = reinterpret_cast<const int32_t*>(ws);
  const int32_t n = hdr[0], S = hdr[1];
  const float* part = ws + kSplitHdrBytes / 4;
  const int64_t work = (int64_t)n * 256 * 64;  // (tile, row, group of 4 columns)
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < work;
       i0 += kReduceItems * stride) {
    v4f acc[kReduceItems];
    int64_t dsto[kReduceItems];
    int32_t pcol[kReduceItems];
#pragma unroll
    for (int u = 0; u < kReduceItems; ++u) {
      const int64_t i = i0 + u * stride;
      dsto[u] = -1;
      pcol[u] = 0;
      acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
      if (i >= work) continue;
      const int32_t t = (int32_t)(i >> 14), r = (int32_t)((i >> 6) & 255),
                    c = (int32_t)(i & 63) * 4;
      const int32_t* th = hdr + 4 + 4 * t;
      const int32_t q = th[0] + r, p = th[1] + c;
      if (q < th[2] || q >= th[3] || p >= N) continue;
      dsto[u] = (int64_t)q * ldo + p;
      pcol[u] = p;
      const float* src = part + (int64_t)t * S * 65536 + r * 256 + c;
      acc[u] = *reinterpret_cast<const v4f*>(src);
      for (int32_t sp = 1; sp < S; ++sp)
        acc[u] += *reinterpret_cast<const v4f*>(src + (int64_t)sp * 65536);
    }
#pragma unroll
    for (int u = 0; u < kReduceItems; ++u) {
      if (dsto[u] < 0) continue;
      const int32_t p = pcol[u];
      if (out_f32) {
        float* dst = reinterpret_cast<float*>(out) + dsto[u];
        if (p + 4 <= N)
          *reinterpret_cast<v4f*>(dst) = acc[u];
        else
          for (int32_t k = 0; p + k < N; ++k) dst[k] = acc[u][k];
      } else {
        uint16_t* dst = reinterpret_cast<uint16_t*>(out) + dsto[u];
        if (p + 4 <= N) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(acc[u][0], acc[u][1]),
                                                      pack_bf16x2(acc[u][2], acc[u][3]));
        } else {
          for (int32_t k = 0; p + k < N; ++k) {
            const __bf16 h = (__bf16)acc[u][k];
            dst[k] = *reinterpret_cast<const uint16_t*>(&h);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wgrad: dw[g][n][k] = sum_{t in g} go[n][t] ia[k][t].  Experts are visited
// largest-first so the longest contraction runs start in the first round.
// With split-K (args.split > 0 tokens, fp32 output zeroed by the caller) an
// expert's tokens are cut into chunks of args.split, every (chunk, tile) is
// one work item, and the partial sums are added with fp32 atomics; empty
// experts then produce no work (their zeros are already in place).
// ---------------------------------------------------------------------------
template <bool SCALED, bool F32>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_wgrad(WgradArgs args, uint32_t gm) {
  __shared__ Smem sm;
  const int E = args.E;
  const int32_t M = args.M;
  const int32_t split = args.split;
  // sizes into sched[0..E-1], then rank experts by descending size (ties by index)
  monotone_ends_to_lds(args.group_ends, E, M, sm.gend);
  for (int g = threadIdx.x; g < E; g += kThreads) {
    int32_t b, e;
    group_range(sm.gend, g, b, e);
    sm.sched[g] = e - b;
  }
  __syncthreads();
  const uint32_t n_tiles = ((uint32_t)args.N + kTileQ - 1) / kTileQ;  // Q = go rows (n)
  const uint32_t k_tiles = ((uint32_t)args.K + kTileP - 1) / kTileP;  // P = ia rows (k)
  const uint32_t per_expert = n_tiles * k_tiles;
  for (int g = threadIdx.x; g < E; g += kThreads) {
    const int32_t sg = sm.sched[g];
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const int32_t sj = sm.sched[j];
      rank += (sj > sg) || (sj == sg && j < g);
    }
    sm.order[rank] = g;
    const int32_t c = split > 0 ? (sg + split - 1) / split : 1;
    sm.chunks[rank] = c;
  }
  __syncthreads();
  // work items per rank -> prefix in sm.items (sched is free again: reuse it
  // as the scan input)
  for (int r = threadIdx.x; r < E; r += kThreads) sm.sched[r] = sm.chunks[r] * (int32_t)per_expert;
  __syncthreads();
  scan_counts(sm, sm.sched, sm.items, E);
  const uint32_t total = (uint32_t)sm.items[E];
  const bool staged = split > 0 && args.split_ws != nullptr;
  if (staged && blockIdx.x == 0) {
    int32_t* hdr = reinterpret_cast<int32_t*>(args.split_ws);
    if (threadIdx.x == 0) {
      hdr[0] = E;
      hdr[1] = (int32_t)per_expert;
      hdr[2] = (int32_t)n_tiles;
      hdr[3] = (int32_t)k_tiles;
      hdr[4] = (int32_t)gm;
    }
    for (int r = threadIdx.x; r < E; r += kThreads) {
      hdr[8 + 4 * r] = sm.order[r];
      hdr[9 + 4 * r] = sm.items[r];
      hdr[10 + 4 * r] = sm.chunks[r];
    }
  }

  for (uint32_t base = 0;; base += gridDim.x) {
    const uint32_t lid = xcd_slice(base);
    if (lid >= total) break;
    // rank of item lid: last r with items[r] <= lid
    const int rank = last_le(sm.items, E, lid);
    const int g = sm.order[rank];
    const uint32_t local = lid - (uint32_t)sm.items[rank];
    const uint32_t chunk = local / per_expert;  // consecutive items share a token range
    uint32_t nt, kt;
    band_decode(local - chunk * per_expert, n_tiles, k_tiles, gm, nt, kt);
    int32_t tb, te;
    group_range(sm.gend, g, tb, te);
    int32_t cb = tb, ce = te;
    if (split > 0) {
      cb = tb + (int32_t)chunk * split;
      ce = min(te, cb + split);
    }
    const uint32_t q0 = nt * kTileQ;
    const uint32_t p0 = kt * kTileP;

    Operand P, Q;
    P.data = make_desc(args.ia, (uint32_t)((int64_t)(args.K - 1) * args.ldia + M));
    P.ld = (uint32_t)args.ldia;
    P.row0 = p0;
    P.hi = 128u;
    Q.data = make_desc(args.go, (uint32_t)((int64_t)(args.N - 1) * args.ldgo + M));
    Q.ld = (uint32_t)args.ldgo;
    Q.row0 = q0;
    Q.hi = 128u;
    if (SCALED) {
      P.scale = make_desc(args.ias, scale_extent(M / 32, args.ldias, args.K));
      P.lds = (uint32_t)args.ldias;
      Q.scale = make_desc(args.gos, scale_extent(M / 32, args.ldgos, args.N));
      Q.lds = (uint32_t)args.ldgos;
    }
    // The dW tile: a partial of a split expert into the workspace, or the
    // expert's slice of dW.
    auto finish = [&](const v4f (&acc)[64]) {
      if (staged && sm.chunks[rank] > 1) {
        // one of several partials of this tile: the whole fp32 256x256 block
        char* slot = reinterpret_cast<char*>(args.split_ws) + kWgHdrBytes +
                     (int64_t)lid * kPartialBytes;
        epilogue<true>(sm, acc, slot, 1024, 0u, 0u, 256u, 0u, 256u);
        return;
      }
      char* out = reinterpret_cast<char*>(args.dw) + (int64_t)g * args.ldw_e * (F32 ? 4 : 2);
      if constexpr (F32)
        epilogue<true>(sm, acc, out, args.ldw_n * 4, q0, 0u, (uint32_t)args.N, p0,
                       (uint32_t)args.K, split > 0 && !staged);
      else
        epilogue_bf16(sm, acc, out, args.ldw_n * 2, q0, 0u, (uint32_t)args.N, p0,
                      (uint32_t)args.K);
    };
    // Each path keeps its own accumulators: shared ones made the register
    // allocator copy accumulators inside the unmasked loop of the unscaled
    // kernel.
    if (SCALED && ((tb | te) & 31) != 0) {
      // A group boundary inside a 32-token block breaks the block/scale
      // pairing: the whole expert is written as NaN rather than a wrong value.
      v4f acc[64];
#pragma unroll
      for (int i = 0; i < 64; ++i) acc[i] = v4f{1.0f, 1.0f, 1.0f, 1.0f} * __builtin_nanf("");
      finish(acc);
    } else if (!SCALED && ((cb | ce) & 15) != 0) {
      // unscaled, token range off the 16-byte load grid: masked to the token
      v4f acc[64];
      mainloop<false, true>(sm, P, Q, (uint32_t)cb, (uint32_t)ce, acc);
      finish(acc);
    } else {
      v4f acc[64];
      mainloop<SCALED>(sm, P, Q, (uint32_t)cb, (uint32_t)ce, acc);
      finish(acc);
    }
  }
}

// dW tiles of experts whose tokens were cut into several chunks: the chunks'
// fp32 partials added in chunk order (the first is the starting value);
// experts without tokens (no work items) written as zeros; experts with one
// chunk were written by the GEMM itself.  Items are (rank, tile, row,
// 4-column group), 4 per thread a grid-stride apart, loads before adds.
__global__ __launch_bounds__(256) void k_wgrad_split_reduce(const float* __restrict__ ws,
                                                            void* __restrict__ dw, int32_t N,
                                                            int32_t K, int64_t ldw_e,
                                                            int64_t ldw_n, int32_t out_f32) {
  const int32_t* hdr = reinterpret_cast<const int32_t*>(ws);
  const int32_t E = hdr[0], per_expert = hdr[1], n_tiles = hdr[2], k_tiles = hdr[3];
  const uint32_t gm = (uint32_t)hdr[4];
  const float* part = ws + kWgHdrBytes / 4;
  const int64_t per_rank = (int64_t)per_expert * 16384;
  const int64_t work = (int64_t)E * per_rank;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < work;
       i0 += kReduceItems * stride) {
    v4f acc[kReduceItems];
    int64_t dsto[kReduceItems];
    int32_t pcol[kReduceItems];
#pragma unroll
    for (int u = 0; u < kReduceItems; ++u) {
      const int64_t i = i0 + u * stride;
      dsto[u] = -1;
      pcol[u] = 0;
      acc[u] = v4f{0.f, 0.f, 0.f, 0.f};
      if (i >= work) continue;
      const int32_t r = (int32_t)(i / per_rank);
      const int32_t t = (int32_t)((i >> 14) % per_expert);
      const int32_t row = (int32_t)((i >> 6) & 255), c = (int32_t)(i & 63) * 4;
      const int32_t* rh = hdr + 8 + 4 * r;
      const int32_t chunks = rh[2];
      if (chunks == 1) continue;
      uint32_t nt, kt;
      band_decode((uint32_t)t, (uint32_t)n_tiles, (uint32_t)k_tiles, gm, nt, kt);
      const int32_t n = (int32_t)nt * 256 + row, k = (int32_t)kt * 256 + c;
      if (n >= N || k >= K) continue;
      dsto[u] = (int64_t)rh[0] * ldw_e + (int64_t)n * ldw_n + k;
      pcol[u] = k;
      if (chunks == 0) continue;
      const float* src = part + ((int64_t)rh[1] + t) * 65536 + row * 256 + c;
      acc[u] = *reinterpret_cast<const v4f*>(src);
      for (int32_t ch = 1; ch < chunks; ++ch)
        acc[u] += *reinterpret_cast<const v4f*>(src + (int64_t)ch * per_expert * 65536);
    }
#pragma unroll
    for (int u = 0; u < kReduceItems; ++u) {
      if (dsto[u] < 0) continue;
      const int32_t k = pcol[u];
      if (out_f32) {
        float* dst = reinterpret_cast<float*>(dw) + dsto[u];
        if (k + 4 <= K)
          *reinterpret_cast<v4f*>(dst) = acc[u];
        else
          for (int32_t j = 0; k + j < K; ++j) dst[j] = acc[u][j];
      } else {
        uint16_t* dst = reinterpret_cast<uint16_t*>(dw) + dsto[u];
        if (k + 4 <= K) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(acc[u][0], acc[u][1]),
                                                      pack_bf16x2(acc[u][2], acc[u][3]));
        } else {
          for (int32_t j = 0; k + j < K; ++j) {
            const __bf16 h = (__bf16)acc[u][j];
            dst[j] = *reinterpret_cast<const uint16_t*>(&h);
          }
        }
      }
    }
  }
}

int persistent_grid() {
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  return (cus + 7) / 8 * 8;
}

}  // namespace

int64_t wgrad_split_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t E, int64_t split) {
  // sum over experts of ceil(tokens / split) <= M / split + E
  const int64_t tiles = ((N + 255) / 256) * ((K + 255) / 256);
  return kWgHdrBytes + (M / split + E) * tiles * kPartialBytes;
}

int64_t fwd_split_workspace_bytes() {
  return kSplitHdrBytes + (int64_t)persistent_grid() * kPartialBytes;
}

// Scratch of the allocation-free forward split (mxgg_grouped_fwd_split_noalloc):
// the split header and one fp32 256x256 partial per workgroup of a persistent
// grid of up to kNoallocUnits workgroups.  Every device holds its own copy
// until the process ends.  In host code `scratch` only names the symbol: the
// device address comes from hipGetSymbolAddress, once per device.
constexpr int64_t kNoallocUnits = 256;
constexpr int64_t kNoallocScratchBytes = kSplitHdrBytes + kNoallocUnits * kPartialBytes;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

int64_t noalloc_scratch_bytes() { return kNoallocScratchBytes; }

void* noalloc_scratch() {
  static std::mutex mu;
  static std::vector<void*> ptrs;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)ptrs.size() <= dev) ptrs.resize(dev + 1, nullptr);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

hipError_t launch_grouped_fwd(const FwdArgs& a, hipStream_t stream) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  const dim3 grid(persistent_grid()), block(kThreads);
  const uint32_t gm = 8;
  const bool keep = a.out != nullptr;
  const int out = a.swiglu_mode == MXGG_SCALE_RCEIL   ? (keep ? kOutSwigluKeepRceil : kOutSwigluRceil)
                  : a.swiglu_mode == MXGG_SCALE_FLOOR ? (keep ? kOutSwigluKeepFloor : kOutSwigluFloor)
                  : a.out_f32                         ? kOutF32
                                                      : kOutBf16;
#define MXGG_FWD(S, O) hipLaunchKernelGGL((k_grouped_fwd<S, O>), grid, block, 0, stream, a, gm)
#define MXGG_FWD_OUT(S)                                           \
  switch (out) {                                                  \
    case kOutF32: MXGG_FWD(S, kOutF32); break;                    \
    case kOutSwigluRceil: MXGG_FWD(S, kOutSwigluRceil); break;    \
    case kOutSwigluFloor: MXGG_FWD(S, kOutSwigluFloor); break;    \
    case kOutSwigluKeepRceil: MXGG_FWD(S, kOutSwigluKeepRceil); break; \
    case kOutSwigluKeepFloor: MXGG_FWD(S, kOutSwigluKeepFloor); break; \
    default: MXGG_FWD(S, kOutBf16); break;                        \
  }
  if (a.scaled) {
    MXGG_FWD_OUT(true)
  } else {
    MXGG_FWD_OUT(false)
  }
#undef MXGG_FWD_OUT
#undef MXGG_FWD
  if (a.split_ws == nullptr) return hipGetLastError();
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(k_fwd_split_reduce, dim3(4 * grid.x), dim3(256), 0, stream, a.split_ws,
                     a.out, a.ldo, a.N, a.out_f32);
  return hipGetLastError();
}

hipError_t launch_grouped_wgrad(const WgradArgs& a, hipStream_t stream) {
  if (a.N == 0 || a.K == 0 || a.E == 0) return hipSuccess;
  const dim3 grid(persistent_grid()), block(kThreads);
  const uint32_t gm = 4;
#define MXGG_WG(S, F) hipLaunchKernelGGL((k_grouped_wgrad<S, F>), grid, block, 0, stream, a, gm)
  if (a.scaled) {
    if (a.out_f32) MXGG_WG(true, true); else MXGG_WG(true, false);
  } else {
    if (a.out_f32) MXGG_WG(false, true); else MXGG_WG(false, false);
  }
#undef MXGG_WG
  if (a.split <= 0 || a.split_ws == nullptr) return hipGetLastError();
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(k_wgrad_split_reduce, dim3(4 * grid.x), dim3(256), 0, stream, a.split_ws,
                     a.dw, a.N, a.K, a.ldw_e, a.ldw_n, a.out_f32);
  return hipGetLastError();
}

}  // namespace mxgg
