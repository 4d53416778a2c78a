// MXFP8 grouped GEMM kernels for gfx950 (CDNA4) on v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Both kernels compute tiles of
//   D[p][q] = sum_k P[p][k] * 2^(sP[k/32][p]-127) * Q[q][k] * 2^(sQ[k/32][q]-127)
// where P and Q are row-major e4m3 operands contiguous along the contraction
// dimension k and the E8M0 scales are stored block-major (one row of bytes per
// 32-deep k-block, indexed by operand row).  P feeds the MFMA "A" source (its
// index lands on the 4 consecutive accumulator rows each lane holds), Q feeds
// the "B" source (one index per lane), so the output's contiguous dimension is
// the P index.
//
//   forward : P = W[g] (rows n), Q = X (rows m of group g), k = hidden  -> Y[m][n]
//   wgrad   : P = X^T  (rows k), Q = dY^T (rows n),  k = tokens of g    -> dW[g][n][k]
//
// Tile 256(P) x 256(Q), 256 threads = 4 waves in a 2x2 arrangement, each wave
// 128x128 = 4x4 MFMA 32x32 blocks (256 fp32 accumulators per lane in AGPRs).
// The contraction streams through a ring of 4 LDS stages of 64 (two k-blocks):
// each stage holds P and Q (256 rows x 64 B each, 16-byte chunks XOR-swizzled
// per row) and their 4 scale rows, all written by LDS-DMA
// (buffer_load ... lds) three stages ahead of the compute.  Each stage's MFMA
// sequence is split around the barrier that publishes the next stage: the
// last 8 MFMAs of stage s run while the waves synchronise and read stage s+1's
// operands, so the matrix pipe does not drain at stage boundaries.
// Persistent grid (one workgroup per CU), tiles dealt round-robin with each XCD
// taking a contiguous slice of every round.
#include <algorithm>

#include "mxgg_internal.h"

namespace mxgg {
namespace {

constexpr int kTileP = 256;
constexpr int kTileQ = 256;
constexpr int kStageK = 64;     // contraction elements (bytes) per stage
constexpr int kStages = 4;      // LDS ring depth
constexpr int kAhead = 3;       // stages in flight ahead of the compute
constexpr int kThreads = 256;
constexpr int kMaxGroups = 1024;
constexpr uint32_t kOpBytes = 256u * kStageK;          // one operand of one stage: 16 KB
constexpr uint32_t kScaleOff = 2u * kOpBytes;          // scale rows after P and Q data
constexpr uint32_t kStageBytes = 2u * kOpBytes + 1024u;  // + [2 operands][2 blocks][256]
// DMA instructions per wave per stage: 4 P + 4 Q (+ 1 scale when scaled)
template <bool SCALED>
constexpr uint32_t dma_per_stage() { return SCALED ? 9u : 8u; }
constexpr uint32_t kOobOffset = 0x80000000u;           // beyond every num_records we create

struct __align__(16) Smem {
  uint8_t ring[kStages][kStageBytes];
  int32_t sched[kMaxGroups + 1];
  int32_t order[kMaxGroups];
  int32_t scan_tmp[kThreads];
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

struct Operand {
  desc_t data;    // [rows][ld] e4m3
  desc_t scale;   // [k-blocks][lds] E8M0, block-major
  uint32_t ld;    // bytes per data row
  uint32_t lds;   // bytes per scale block-row (multiple of 4)
  uint32_t row0;  // first operand row of this tile (multiple of 4)
  uint32_t rows;  // rows that exist (data loads clamp to rows-1)
};

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t wave_id() {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Byte offset of a __shared__ object inside the workgroup's LDS allocation.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)((const lds_void_t*)p);
}

// 16-byte chunk swizzle inside a 64-byte LDS row.  For 8 consecutive rows the
// (row parity, chunk) pairs are distinct (conflict-free 8-lane service of a
// 32-bank LDS) and for 16 consecutive rows the (row mod 4, chunk) pairs are
// distinct (16-lane service of a 64-bank LDS).
__device__ __forceinline__ uint32_t swz(uint32_t r) { return ((r >> 1) ^ (r >> 3)) & 3u; }

// Publish a stage: this wave's DMA older than the 2 youngest stages (18
// instructions scaled, 16 unscaled) has landed and all of its LDS reads have
// returned, then the workgroup barrier.  Written as assembly so the
// compiler's waitcnt pass can neither relax nor move it (it does not see the
// DMA, and would drop the lgkmcnt part for reads whose results are only used
// after the barrier).
template <bool SCALED>
__device__ __forceinline__ void publish_barrier() {
  static_assert((kAhead - 1) * dma_per_stage<SCALED>() == (SCALED ? 18u : 16u),
                "wait counts below are written out for 2 stages in flight");
  if (SCALED)
    asm volatile("s_waitcnt vmcnt(18) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}


// LDS-DMA issued from inline assembly: M0 holds the wave's LDS destination,
// each lane its byte offset into the buffer.  The compiler does not track
// these loads, so it inserts no wait for them in front of LDS reads of other
// stages; every consumer waits explicitly in publish_barrier().
// M0 is reserved by the compiler, which warns about the clobber; on gfx950 it
// only uses M0 for LDS-DMA, GWS and message instructions, none of which it
// emits in these kernels (the generated code writes M0 only here).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_x4(const desc_t& d, uint32_t lds_addr, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds_addr), "v"(voff), "s"(d)
      : "memory", "m0");
}
__device__ __forceinline__ void dma_x1(const desc_t& d, uint32_t lds_addr, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(lds_addr), "v"(voff), "s"(d)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// Per-thread state of the global -> LDS stream for one tile.
//  Data: wave w's i-th load (i = 0..3) fills LDS bytes [(4i+w)*1024, +1024) of
//  an operand, lane l writing 16 B at +16*l: LDS row r = (4i+w)*16 + l/4 at
//  physical chunk l%4, so the lane fetches logical chunk (l%4) ^ swz(r) of
//  operand row r.  swz(r) does not depend on i, so one chunk column serves all
//  four loads.  Chunks at or past kend are fetched from an out-of-range offset
//  and land as zeros.
//  Scales: wave w copies block (w&1) of operand (w>>1): 256 rows = 64 lanes x
//  4 bytes, from block-row kb + (w&1).  A block at or past kend lands as zeros
//  (scale 2^-127 on zero payload).
template <bool SCALED>
struct Stream {
  uint32_t offp[4], offq[4];
  uint32_t kcol;
  uint32_t soff;   // this wave's scale source offset within a block-row
  uint32_t slds;   // this wave's scale destination inside a stage

  __device__ __forceinline__ void init(const Operand& P, const Operand& Q) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = wave_id();
    const uint32_t c = (lane & 3u) ^ swz(wave * 16u + (lane >> 2));
    kcol = 16u * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = (4u * i + wave) * 16u + (lane >> 2);
      offp[i] = min(P.row0 + r, P.rows - 1u) * P.ld + kcol;
      offq[i] = min(Q.row0 + r, Q.rows - 1u) * Q.ld + kcol;
    }
    if (SCALED) {
      const Operand& X = (wave >> 1) ? Q : P;
      soff = X.row0 + 4u * lane;
      slds = kScaleOff + (wave >> 1) * 512u + (wave & 1u) * 256u;
    }
  }

  __device__ __forceinline__ void issue(uint8_t* stage, const Operand& P, const Operand& Q,
                                        uint32_t k0, uint32_t kend) {
    const uint32_t wave = wave_id();
    const uint32_t base = lds_offset(stage) + wave * 1024u;
    const bool ok = k0 + kcol < kend;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_x4(P.data, base + 4096u * i, ok ? offp[i] + k0 : kOobOffset);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma_x4(Q.data, base + kOpBytes + 4096u * i, ok ? offq[i] + k0 : kOobOffset);
    if (SCALED) {
      const uint32_t blk = (k0 >> 5) + (wave & 1u);
      const Operand& X = (wave >> 1) ? Q : P;
      const uint32_t off = (blk < (kend >> 5)) ? blk * X.lds + soff : kOobOffset;
      dma_x1(X.scale, lds_offset(stage) + slds, off);
    }
  }
};

// Operands of one stage in registers: 4 P fragments, 4 Q fragments, their scales.
struct Frags {
  v8i a[4], b[4];
  uint32_t sa[4], sb[4];
};

// Per-lane LDS byte offsets (relative to a stage) of fragment 0; fragment i
// adds 32 rows = 2048 bytes, its scale 32 bytes.
//   v_mfma_scale_f32_32x32x64_f8f6f4 (fp8) operand layout: lane l serves row
//   l%32; its bytes 0..15 belong to scale block 0 and bytes 16..31 to block 1
//   of the 64-deep step, both halves of the wave sharing each block, and the
//   block-b scale of row r comes from lane r + 32b.  So lane half h takes
//   chunk h (of block 0: chunks 0,1) and chunk 2+h (of block 1: chunks 2,3),
//   and the scale byte of block h.
struct FragAddr {
  uint32_t plo, phi, qlo, qhi, ps, qs;

  __device__ __forceinline__ void init() {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t wp = wave & 1u, wq = wave >> 1;
    const uint32_t l32 = lane & 31u, h = lane >> 5;
    const uint32_t rp = wp * 128u + l32, rq = wq * 128u + l32;
    // swz(r + 32i) == swz(r): adding 32 rows changes neither (r>>1)&3 nor (r>>3)&3
    plo = rp * kStageK + ((h ^ swz(rp)) << 4);
    phi = rp * kStageK + (((2u + h) ^ swz(rp)) << 4);
    qlo = kOpBytes + rq * kStageK + ((h ^ swz(rq)) << 4);
    qhi = kOpBytes + rq * kStageK + (((2u + h) ^ swz(rq)) << 4);
    ps = kScaleOff + h * 256u + rp;
    qs = kScaleOff + 512u + h * 256u + rq;
  }
};

__device__ __forceinline__ v8i lds_v8i(const uint8_t* lo, const uint8_t* hi) {
  const uint4 a = *reinterpret_cast<const uint4*>(lo);
  const uint4 b = *reinterpret_cast<const uint4*>(hi);
  v8i f;
  f[0] = (int)a.x; f[1] = (int)a.y; f[2] = (int)a.z; f[3] = (int)a.w;
  f[4] = (int)b.x; f[5] = (int)b.y; f[6] = (int)b.z; f[7] = (int)b.w;
  return f;
}

// Fragment reads are split so they spread over the MFMA stream:
//   head : Q fragments 0..3, P fragments 0..1 and all scale bytes of a stage
//   tail : P fragments 2..3
template <bool SCALED>
__device__ __forceinline__ void read_head(const uint8_t* stage, const FragAddr& fa, Frags& f) {
#pragma unroll
  for (int j = 0; j < 4; ++j) f.b[j] = lds_v8i(stage + fa.qlo + 2048u * j, stage + fa.qhi + 2048u * j);
#pragma unroll
  for (int i = 0; i < 2; ++i) f.a[i] = lds_v8i(stage + fa.plo + 2048u * i, stage + fa.phi + 2048u * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f.sa[i] = SCALED ? (uint32_t)stage[fa.ps + 32u * i] : 127u;
    f.sb[i] = SCALED ? (uint32_t)stage[fa.qs + 32u * i] : 127u;
  }
}

__device__ __forceinline__ void read_tail(const uint8_t* stage, const FragAddr& fa, Frags& f) {
#pragma unroll
  for (int i = 2; i < 4; ++i) f.a[i] = lds_v8i(stage + fa.plo + 2048u * i, stage + fa.phi + 2048u * i);
}

__device__ __forceinline__ void mfma_row(const Frags& f, int i, v16f (&acc)[4][4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.a[i], f.b[j], acc[i][j], 0, 0, 0,
                                                               (int)f.sa[i], 0, (int)f.sb[j]);
}

// One stage s: issue the DMA of stage s+kAhead, read P fragments 2..3 of
// stage s, MFMA rows 0..1, wait for stage s+1's DMA (the two younger stages
// stay in flight) and for this wave's LDS reads, barrier, read the head of
// stage s+1 into `nxt`, then MFMA rows 2..3, which overlap the barrier and the
// reads.  The step has no branches: the DMA of stages past the end is issued
// anyway (it lands as zeros in a slot nobody reads again), so the wait count
// is a constant, and after the last stage the head read fetches a stale slot
// that is never used.
template <bool SCALED>
__device__ __forceinline__ void stage_step(Smem& sm, Stream<SCALED>& st, const Operand& P,
                                           const Operand& Q, const FragAddr& fa, Frags& cur,
                                           Frags& nxt, uint32_t s, uint32_t kbeg, uint32_t kend,
                                           v16f (&acc)[4][4]) {
  st.issue(sm.ring[(s + kAhead) % kStages], P, Q, kbeg + (s + kAhead) * kStageK, kend);
  read_tail(sm.ring[s % kStages], fa, cur);
  __builtin_amdgcn_sched_barrier(0);
  mfma_row(cur, 0, acc);
  mfma_row(cur, 1, acc);
  __builtin_amdgcn_sched_barrier(0);
  publish_barrier<SCALED>();
  __builtin_amdgcn_sched_barrier(0);
  read_head<SCALED>(sm.ring[(s + 1) % kStages], fa, nxt);
  mfma_row(cur, 2, acc);
  mfma_row(cur, 3, acc);
  __builtin_amdgcn_sched_barrier(0);
}

template <bool SCALED>
__device__ __forceinline__ void mainloop(Smem& sm, const Operand& P, const Operand& Q,
                                         uint32_t kbeg, uint32_t kend, v16f (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  if (kend <= kbeg) return;
  // The loop body computes two stages; an odd stage count gets one extra
  // stage past kend, which the DMA fills with zero payload and zero scale
  // bytes, adding exactly nothing.  (A conditional tail stage would make the
  // accumulators live across a branch and spill.)
  const uint32_t nsteps = ((kend - kbeg + 2 * kStageK - 1) / (2 * kStageK)) * 2;
  Stream<SCALED> st;
  st.init(P, Q);
  FragAddr fa;
  fa.init();
  // Prologue: stages 0 .. kAhead-1 in flight, then publish stage 0.
#pragma unroll
  for (uint32_t s = 0; s < (uint32_t)kAhead; ++s)
    st.issue(sm.ring[s], P, Q, kbeg + s * kStageK, kend);
  publish_barrier<SCALED>();
  __builtin_amdgcn_sched_barrier(0);
  Frags f0, f1;
  read_head<SCALED>(sm.ring[0], fa, f0);
  // Stage s+kAhead goes into the ring slot of stage s-1, which every wave
  // finished reading before the barrier inside step s-1.
  for (uint32_t s = 0; s < nsteps; s += 2) {
    stage_step<SCALED>(sm, st, P, Q, fa, f0, f1, s, kbeg, kend, acc);
    stage_step<SCALED>(sm, st, P, Q, fa, f1, f0, s + 1, kbeg, kend, acc);
  }
  // Drain the DMA of the stages past the end before the next tile's prologue
  // reuses the ring.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const __bf16 ha = (__bf16)a, hb = (__bf16)b;
  const uint16_t ua = *reinterpret_cast<const uint16_t*>(&ha);
  const uint16_t ub = *reinterpret_cast<const uint16_t*>(&hb);
  return (uint32_t)ua | ((uint32_t)ub << 16);
}

// Store the 4 consecutive outputs (P index p..p+3) of accumulator quad rg of
// block (i, j) for this lane's Q index.  `rowp` points at element [q][0].
template <bool F32>
__device__ __forceinline__ void store4(void* rowp, uint32_t p, uint32_t pend, const v16f& a,
                                       int rg) {
  const float v0 = a[4 * rg + 0], v1 = a[4 * rg + 1], v2 = a[4 * rg + 2], v3 = a[4 * rg + 3];
  if (F32) {
    float* d = reinterpret_cast<float*>(rowp) + p;
    if (p + 3 < pend) {
      *reinterpret_cast<float4*>(d) = make_float4(v0, v1, v2, v3);
    } else {
      const float v[4] = {v0, v1, v2, v3};
      for (int u = 0; u < 4; ++u)
        if (p + u < pend) d[u] = v[u];
    }
  } else {
    uint16_t* d = reinterpret_cast<uint16_t*>(rowp) + p;
    if (p + 3 < pend) {
      *reinterpret_cast<uint2*>(d) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
    } else {
      const float v[4] = {v0, v1, v2, v3};
      for (int u = 0; u < 4; ++u)
        if (p + u < pend) {
          const __bf16 hv = (__bf16)v[u];
          d[u] = *reinterpret_cast<const uint16_t*>(&hv);
        }
    }
  }
}

// Write the tile: output row = Q index in [qbeg, qend), column = P index < pend.
template <bool F32>
__device__ __forceinline__ void epilogue(const v16f (&acc)[4][4], char* out, int64_t ldo_bytes,
                                         uint32_t q0, uint32_t qbeg, uint32_t qend, uint32_t p0,
                                         uint32_t pend) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t wp = wave & 1u, wq = wave >> 1;
  const uint32_t l32 = lane & 31u, h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t q = q0 + wq * 128u + 32u * j + l32;
    if (q < qbeg || q >= qend) continue;
    char* rowp = out + (int64_t)q * ldo_bytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const uint32_t p = p0 + wp * 128u + 32u * i + 8u * rg + 4u * h;
        if (p < pend) store4<F32>(rowp, p, pend, acc[i][j], rg);
      }
    }
  }
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

// Position in the global tile order processed by this workgroup at round
// `base`: each XCD (workgroups are dealt to the 8 XCDs round-robin) takes a
// contiguous slice of the round.
__device__ __forceinline__ uint32_t xcd_slice(uint32_t base) {
  const uint32_t g = gridDim.x;  // multiple of 8
  return base + (blockIdx.x & 7u) * (g >> 3) + (blockIdx.x >> 3);
}

// Block-wide inclusive scan of per-group tile counts into sm.sched[1..E]
// (sched[0] = 0).  Each thread owns 4 consecutive groups.
__device__ void scan_tiles(Smem& sm, const int32_t* tiles_of /*LDS, E*/, int E) {
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
    if (g < E) sm.sched[g + 1] = run;
  }
  if (t == 0) sm.sched[0] = 0;
  __syncthreads();
}

__device__ __forceinline__ void group_range(const int32_t* ends, int g, int32_t limit,
                                            int32_t& beg, int32_t& end) {
  int32_t e = ends[g];
  int32_t b = g > 0 ? ends[g - 1] : 0;
  e = e < 0 ? 0 : (e > limit ? limit : e);
  b = b < 0 ? 0 : (b > limit ? limit : b);
  beg = b;
  end = e > b ? e : b;
}

// ---------------------------------------------------------------------------
// Forward: out[m][n] = sum_k A[m][k] W[g][n][k] for m in group g.  The m-tiles
// of a group start at the group's first row rounded down to a multiple of 4
// (the scale DMA copies 4 rows per lane); rows outside the group are computed
// but not stored.
// ---------------------------------------------------------------------------
template <bool SCALED, bool F32>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_fwd(FwdArgs args, uint32_t gm) {
  __shared__ Smem sm;
  const int E = args.group_ends ? args.E : 1;
  const int32_t M = args.M;
  for (int g = threadIdx.x; g < E; g += kThreads) {
    int32_t b = 0, e = M;
    if (args.group_ends) group_range(args.group_ends, g, M, b, e);
    sm.order[g] = e > b ? (e - (b & ~3) + kTileQ - 1) / kTileQ : 0;
  }
  __syncthreads();
  scan_tiles(sm, sm.order, E);
  const uint32_t m_tiles = (uint32_t)sm.sched[E];
  const uint32_t n_tiles = ((uint32_t)args.N + kTileP - 1) / kTileP;
  const uint32_t total = m_tiles * n_tiles;
  const uint32_t K = (uint32_t)args.K;

  for (uint32_t base = 0;; base += gridDim.x) {
    const uint32_t lid = xcd_slice(base);
    if (lid >= total) break;
    uint32_t mt, nt;
    band_decode(lid, m_tiles, n_tiles, gm, mt, nt);
    // group of m-tile mt: last g with sched[g] <= mt
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((uint32_t)sm.sched[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    const int g = lo;
    int32_t gb = 0, ge = M;
    if (args.group_ends) group_range(args.group_ends, g, M, gb, ge);
    const uint32_t q0 = (uint32_t)(gb & ~3) + (mt - (uint32_t)sm.sched[g]) * kTileQ;
    const uint32_t p0 = nt * kTileP;

    Operand P, Q;
    const uint8_t* wg = args.w + (int64_t)g * args.w_gstride;
    P.data = make_desc(wg, (uint32_t)((int64_t)(args.N - 1) * args.ldw + K));
    P.ld = (uint32_t)args.ldw;
    P.row0 = p0;
    P.rows = (uint32_t)args.N;
    Q.data = make_desc(args.a, (uint32_t)((int64_t)(M - 1) * args.lda + K));
    Q.ld = (uint32_t)args.lda;
    Q.row0 = q0;
    Q.rows = (uint32_t)M;
    if (SCALED) {
      const uint8_t* wsg = args.ws + (int64_t)g * args.ws_gstride;
      P.scale = make_desc(wsg, scale_extent(K / 32, args.ldws, args.N));
      P.lds = (uint32_t)args.ldws;
      Q.scale = make_desc(args.as, scale_extent(K / 32, args.ldas, M));
      Q.lds = (uint32_t)args.ldas;
    }
    v16f acc[4][4];
    mainloop<SCALED>(sm, P, Q, 0u, K, acc);
    const int64_t ldo_bytes = args.ldo * (F32 ? 4 : 2);
    epilogue<F32>(acc, reinterpret_cast<char*>(args.out), ldo_bytes, q0, (uint32_t)gb,
                  (uint32_t)ge, p0, (uint32_t)args.N);
  }
}

// ---------------------------------------------------------------------------
// Wgrad: dw[g][n][k] = sum_{t in g} go[n][t] ia[k][t].  Experts are visited
// largest-first so the longest contraction runs start in the first round.
// ---------------------------------------------------------------------------
template <bool SCALED, bool F32>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_wgrad(WgradArgs args, uint32_t gm) {
  __shared__ Smem sm;
  const int E = args.E;
  const int32_t M = args.M;
  // sizes into sched[0..E-1], then rank experts by descending size (ties by index)
  for (int g = threadIdx.x; g < E; g += kThreads) {
    int32_t b, e;
    group_range(args.group_ends, g, M, b, e);
    sm.sched[g] = e - b;
  }
  __syncthreads();
  for (int g = threadIdx.x; g < E; g += kThreads) {
    const int32_t sg = sm.sched[g];
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const int32_t sj = sm.sched[j];
      rank += (sj > sg) || (sj == sg && j < g);
    }
    sm.order[rank] = g;
  }
  __syncthreads();

  const uint32_t n_tiles = ((uint32_t)args.N + kTileQ - 1) / kTileQ;  // Q = go rows (n)
  const uint32_t k_tiles = ((uint32_t)args.K + kTileP - 1) / kTileP;  // P = ia rows (k)
  const uint32_t per_expert = n_tiles * k_tiles;
  const uint32_t total = per_expert * (uint32_t)E;

  for (uint32_t base = 0;; base += gridDim.x) {
    const uint32_t lid = xcd_slice(base);
    if (lid >= total) break;
    const uint32_t rank = lid / per_expert;
    const int g = sm.order[rank];
    uint32_t nt, kt;
    band_decode(lid - rank * per_expert, n_tiles, k_tiles, gm, nt, kt);
    int32_t tb, te;
    group_range(args.group_ends, g, M, tb, te);
    const uint32_t q0 = nt * kTileQ;
    const uint32_t p0 = kt * kTileP;

    Operand P, Q;
    P.data = make_desc(args.ia, (uint32_t)((int64_t)(args.K - 1) * args.ldia + M));
    P.ld = (uint32_t)args.ldia;
    P.row0 = p0;
    P.rows = (uint32_t)args.K;
    Q.data = make_desc(args.go, (uint32_t)((int64_t)(args.N - 1) * args.ldgo + M));
    Q.ld = (uint32_t)args.ldgo;
    Q.row0 = q0;
    Q.rows = (uint32_t)args.N;
    if (SCALED) {
      P.scale = make_desc(args.ias, scale_extent(M / 32, args.ldias, args.K));
      P.lds = (uint32_t)args.ldias;
      Q.scale = make_desc(args.gos, scale_extent(M / 32, args.ldgos, args.N));
      Q.lds = (uint32_t)args.ldgos;
    }
    v16f acc[4][4];
    if (((tb | te) & 31) != 0) {
      // A group boundary inside a 32-token block breaks the block/scale
      // pairing: the whole expert is written as NaN rather than a wrong value.
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_nanf("");
    } else {
      mainloop<SCALED>(sm, P, Q, (uint32_t)tb, (uint32_t)te, acc);
    }
    char* out = reinterpret_cast<char*>(args.dw) +
                (int64_t)g * args.N * args.K * (F32 ? 4 : 2);
    epilogue<F32>(acc, out, (int64_t)args.K * (F32 ? 4 : 2), q0, 0u, (uint32_t)args.N, p0,
                  (uint32_t)args.K);
  }
}

int persistent_grid() {
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  return (cus + 7) / 8 * 8;
}

}  // namespace

hipError_t launch_grouped_fwd(const FwdArgs& a, hipStream_t stream) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  const dim3 grid(persistent_grid()), block(kThreads);
  const uint32_t gm = 8;
#define MXGG_FWD(S, F) hipLaunchKernelGGL((k_grouped_fwd<S, F>), grid, block, 0, stream, a, gm)
  if (a.scaled) {
    if (a.out_f32) MXGG_FWD(true, true); else MXGG_FWD(true, false);
  } else {
    if (a.out_f32) MXGG_FWD(false, true); else MXGG_FWD(false, false);
  }
#undef MXGG_FWD
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
  return hipGetLastError();
}

}  // namespace mxgg
