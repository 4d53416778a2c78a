// MXFP8 grouped GEMM kernels for gfx950 (CDNA4) on v_mfma_scale_f32_32x32x64_f8f6f4.
//
// Both kernels compute tiles of   D[p][q] = sum_k P[p][k]*2^(sP[p][k/32]-127) * Q[q][k]*2^(sQ[q][k/32]-127)
// where P and Q are row-major e4m3 operands contiguous along the contraction
// dimension k.  P feeds the MFMA "A" source (its index lands on the 4
// consecutive accumulator rows each lane holds), Q feeds the "B" source (one
// index per lane).  The output's contiguous dimension is therefore always the
// P index, so each lane stores 4 (bf16: 8 B) or 4 (f32: 16 B) consecutive
// outputs per accumulator quad.
//
//   forward : P = W[g] (rows n), Q = X (rows m of group g), k = hidden  -> Y[m][n]
//   wgrad   : P = X^T  (rows k), Q = dY^T (rows n),  k = tokens of g    -> dW[g][n][k]
//
// Tile 256(P) x 256(Q) x 128(k) per stage, 256 threads = 4 waves in a 2x2
// arrangement, each wave 128x128 = 4x4 MFMA 32x32 blocks (256 fp32
// accumulators per lane, held in AGPRs).  Two LDS stages of P, Q (16-byte
// chunks XOR-swizzled per row) and their scale words: 132 KB of the 160 KB LDS.
// Persistent grid (one workgroup per CU), tiles dealt round-robin with each XCD
// taking a contiguous run of the tile order so the 8 L2s see disjoint,
// locally-reused working sets.
#include <algorithm>

#include "mxgg_internal.h"

namespace mxgg {
namespace {

constexpr int kTileP = 256;
constexpr int kTileQ = 256;
constexpr int kTileK = 128;
constexpr int kThreads = 256;
constexpr int kMaxGroups = 1024;
constexpr uint32_t kOobOffset = 0x80000000u;  // beyond every num_records we create
constexpr uint32_t kScaleOne = 0x7F7F7F7Fu;   // four E8M0 bytes of value 1.0

struct __align__(16) Smem {
  uint8_t p[2][kTileP * kTileK];
  uint8_t q[2][kTileQ * kTileK];
  uint32_t sp[2][kTileP];
  uint32_t sq[2][kTileQ];
  int32_t sched[kMaxGroups + 1];
  int32_t order[kMaxGroups];
  int32_t scan_tmp[kThreads];
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16-byte chunk swizzle inside a 128-byte LDS row.  Rows r..r+7 land on 8
// distinct chunks and rows r, r+8 differ as well, which keeps ds_read_b128 /
// ds_write_b128 conflict free for both 8- and 16-lane service groups.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r ^ (r >> 3)) & 7u; }

// Raw 128-bit buffer descriptor (gfx9 layout: base, stride, num_records,
// dst_sel/format word) for the inline-asm LDS-DMA loads.
typedef int32_t desc_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ desc_t make_desc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  desc_t d;
  d[0] = (int32_t)(uint32_t)a;
  d[1] = (int32_t)((uint32_t)(a >> 32) & 0xFFFFu);  // stride 0
  d[2] = (int32_t)bytes;
  d[3] = 0x00020000;
  return d;
}

struct Operand {
  desc_t data;
  rsrc_t scale;
  uint32_t ld;    // bytes per data row
  uint32_t lds;   // bytes per scale row
  uint32_t row0;  // first operand row of this tile
  uint32_t rows;  // rows that exist (loads clamp to rows-1)
};

typedef __attribute__((address_space(3))) void lds_void_t;

// Wave index within the workgroup as a scalar (wave-uniform) value.
__device__ __forceinline__ uint32_t wave_id() {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// Byte offset of a __shared__ object inside the workgroup's LDS allocation.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)((const lds_void_t*)p);
}

// Global -> LDS pipeline for one 128-deep stage.  Data tiles go straight to
// LDS with buffer_load_dwordx4 ... lds: wave w's i-th load fills LDS bytes
// [(4i+w)*1024, +1024), lane l writing 16 B at +16*l, i.e. LDS row
// r = (4i+w)*8 + l/8 at physical chunk l%8.  Each lane therefore fetches the
// logical chunk (l%8) ^ swz(r) of operand row r.  Rows past the operand clamp
// to its last row; chunks past the contraction end use an offset beyond the
// buffer's num_records, which the hardware returns as zero.
// Scale words (4 E8M0 bytes = the 4 k-blocks of the stage) go through VGPRs.
// Contraction range [kbeg, kend), both multiples of 32.
template <bool SCALED>
struct Pipeline {
  uint32_t offp[8], offq[8];  // per-lane operand offsets (bytes) of the 8 loads
  uint32_t kcol[2];           // logical byte column of this lane's chunk for even / odd i
  uint32_t soffp, soffq;      // per-thread scale row offsets
  uint32_t wsp, wsq;          // scale words of the stage in flight (raw loads)
  uint32_t left;              // contraction bytes left at the stage start

  __device__ __forceinline__ void init(const Operand& P, const Operand& Q) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = wave_id();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t r = (4u * i + wave) * 8u + (lane >> 3);
      const uint32_t c = (lane & 7u) ^ swz(r);
      const uint32_t gp = min(P.row0 + r, P.rows - 1u);
      const uint32_t gq = min(Q.row0 + r, Q.rows - 1u);
      offp[i] = gp * P.ld + 16u * c;
      offq[i] = gq * Q.ld + 16u * c;
    }
    // r = 32i + 8w + l/8, so swz(r) = (l/8) ^ ((4i + w) & 7) only depends on
    // the parity of i: two chunk columns per lane.
    kcol[0] = 16u * ((lane & 7u) ^ swz(wave * 8u + (lane >> 3)));
    kcol[1] = 16u * ((lane & 7u) ^ swz(32u + wave * 8u + (lane >> 3)));
    if (SCALED) {
      soffp = min(P.row0 + threadIdx.x, P.rows - 1u) * P.lds;
      soffq = min(Q.row0 + threadIdx.x, Q.rows - 1u) * Q.lds;
    }
  }

  // Scale words: 4 consecutive E8M0 bytes (the stage's 4 k-blocks) per row.
  // `aligned` (uniform) says every row's word starts on a 4-byte boundary; a
  // full stage then reads one dword that lies inside the row, otherwise four
  // byte loads, each range-checked on its own.  The words are only consumed
  // after the stage's MFMAs, so their wait never lands in front of the compute.
  __device__ __forceinline__ void load_scales(const Operand& P, const Operand& Q, uint32_t k0,
                                              uint32_t kend, bool aligned) {
    const uint32_t kb = k0 >> 5;
    left = kend - k0;
    if (aligned && left >= 128u) {
      wsp = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(P.scale, soffp + kb, 0, 0);
      wsq = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(Q.scale, soffq + kb, 0, 0);
    } else {
      wsp = 0;
      wsq = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        wsp |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(P.scale, soffp + kb + u, 0, 0)
               << (8 * u);
        wsq |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(Q.scale, soffq + kb + u, 0, 0)
               << (8 * u);
      }
    }
  }

  __device__ __forceinline__ void store_scales(Smem& sm, int buf) {
    if (SCALED) {
      uint32_t p = wsp, q = wsq;
      if (left < 128u) {  // blocks past kend read as 1.0 (their payload is zero)
        const uint32_t keep = (1u << (8u * (left >> 5))) - 1u;
        p = (p & keep) | (kScaleOne & ~keep);
        q = (q & keep) | (kScaleOne & ~keep);
      }
      sm.sp[buf][threadIdx.x] = p;
      sm.sq[buf][threadIdx.x] = q;
    }
  }

  // LDS-DMA of one 1 KB slab: M0 holds the wave's LDS destination, each lane
  // supplies its byte offset into the buffer.  Issued from inline assembly:
  // the compiler then inserts no wait for it before unrelated LDS reads (the
  // stage being computed); drain_and_barrier() waits for it explicitly.
  // M0 is reserved by the compiler, which warns about the clobber; on gfx950
  // it only uses M0 for LDS-DMA, GWS and message instructions, none of which
  // it emits in these kernels (the generated code writes M0 only here).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  __device__ __forceinline__ static void dma16(const desc_t& d, uint32_t lds_addr,
                                               uint32_t voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(lds_addr), "v"(voff), "s"(d)
        : "memory", "m0");
  }
#pragma clang diagnostic pop

  __device__ __forceinline__ void issue(Smem& sm, int buf, const Operand& P, const Operand& Q,
                                        uint32_t k0, uint32_t kend, bool aligned) {
    const uint32_t wave = wave_id();
    if (SCALED) load_scales(P, Q, k0, kend, aligned);
    const bool ok[2] = {k0 + kcol[0] < kend, k0 + kcol[1] < kend};
    const uint32_t pbase = lds_offset(&sm.p[buf][0]) + wave * 1024u;
    const uint32_t qbase = lds_offset(&sm.q[buf][0]) + wave * 1024u;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(P.data, pbase + 4096u * i, ok[i & 1] ? offp[i] + k0 : kOobOffset);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dma16(Q.data, qbase + 4096u * i, ok[i & 1] ? offq[i] + k0 : kOobOffset);
  }

};

// Wait for every outstanding memory operation of this wave (including the
// LDS-DMA loads, which the barrier alone does not cover), then barrier.
__device__ __forceinline__ void drain_and_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// MFMA operand of one lane: two 16-byte chunks (logical chunk indices clo and
// chi of an LDS row).
__device__ __forceinline__ v8i lds_frag(const uint8_t* base, uint32_t row, uint32_t clo,
                                        uint32_t chi) {
  const uint32_t s = swz(row);
  const uint4 lo = *reinterpret_cast<const uint4*>(base + row * kTileK + ((clo ^ s) << 4));
  const uint4 hi = *reinterpret_cast<const uint4*>(base + row * kTileK + ((chi ^ s) << 4));
  v8i f;
  f[0] = (int)lo.x; f[1] = (int)lo.y; f[2] = (int)lo.z; f[3] = (int)lo.w;
  f[4] = (int)hi.x; f[5] = (int)hi.y; f[6] = (int)hi.z; f[7] = (int)hi.w;
  return f;
}

// One 128-deep stage of MFMAs out of LDS buffer `buf`.
template <bool SCALED>
__device__ __forceinline__ void compute_stage(const Smem& sm, int buf, v16f (&acc)[4][4]) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t wp = wave & 1u, wq = wave >> 1;
  const uint32_t l32 = lane & 31u, h = lane >> 5;
  uint32_t sa[4], sb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (SCALED) {
      sa[i] = sm.sp[buf][wp * 128u + 32u * i + l32] >> (8u * h);
      sb[i] = sm.sq[buf][wq * 128u + 32u * i + l32] >> (8u * h);
    } else {
      sa[i] = kScaleOne;
      sb[i] = kScaleOne;
    }
  }
  // Operand layout of v_mfma_scale_f32_32x32x64_f8f6f4 (fp8): lane l serves
  // row l%32; its bytes 0..15 belong to scale block 0 and bytes 16..31 to
  // block 1 of the 64-deep step, both halves of the wave sharing each block,
  // and the block-b scale of row r comes from lane r + 32b.  So for substep s
  // (k-blocks 2s, 2s+1 of the stage) lane half h takes chunk 4s+h of block 2s
  // and chunk 4s+2+h of block 2s+1, and its scale byte is byte 2s+h of the
  // row's scale word: (word >> 8h) with op_sel 2s.
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    v8i fa[4], fb[4];
    const uint32_t clo = 4u * s + h, chi = 4u * s + 2u + h;
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = lds_frag(sm.p[buf], wp * 128u + 32u * i + l32, clo, chi);
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = lds_frag(sm.q[buf], wq * 128u + 32u * j + l32, clo, chi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (s == 0)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 0, 0,
                                                                     0, (int)sa[i], 0, (int)sb[j]);
        else
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb[j], acc[i][j], 0, 0,
                                                                     2, (int)sa[i], 2, (int)sb[j]);
      }
    }
  }
}

template <bool SCALED>
__device__ __forceinline__ void mainloop(Smem& sm, const Operand& P, const Operand& Q,
                                         uint32_t kbeg, uint32_t kend, bool scale_aligned,
                                         v16f (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  if (kend <= kbeg) return;
  const uint32_t nsteps = (kend - kbeg + kTileK - 1) / kTileK;
  Pipeline<SCALED> pl;
  pl.init(P, Q);
  pl.issue(sm, 0, P, Q, kbeg, kend, scale_aligned);
  pl.store_scales(sm, 0);
  drain_and_barrier();
  // Steady state: prefetch stage s+1 into the other buffer while computing s.
  uint32_t s = 0;
  for (; s + 1 < nsteps; ++s) {
    const int buf = s & 1;
    pl.issue(sm, buf ^ 1, P, Q, kbeg + (s + 1) * kTileK, kend, scale_aligned);
    compute_stage<SCALED>(sm, buf, acc);
    __builtin_amdgcn_sched_barrier(0);  // keep the scale assembly behind the MFMAs
    pl.store_scales(sm, buf ^ 1);
    drain_and_barrier();
  }
  compute_stage<SCALED>(sm, s & 1, acc);
  __syncthreads();  // LDS is reused by the next tile's prologue
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

// Write the tile: output row index = Q index (q0 + ...), column = P index.
template <bool F32>
__device__ __forceinline__ void epilogue(const v16f (&acc)[4][4], char* out, int64_t ldo_bytes,
                                         uint32_t q0, uint32_t qend, uint32_t p0, uint32_t pend) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t wp = wave & 1u, wq = wave >> 1;
  const uint32_t l32 = lane & 31u, h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t q = q0 + wq * 128u + 32u * j + l32;
    if (q >= qend) continue;
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

// Decode a position in the tile order into (band-major) (mt, nt): bands of
// `gm` consecutive m-tiles are walked column by column so that neighbouring
// tiles share either their Q rows or their P rows.
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
// Forward: out[m][n] = sum_k A[m][k] W[g][n][k] for m in group g.
// ---------------------------------------------------------------------------
template <bool SCALED, bool F32>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_fwd(FwdArgs args, uint32_t gm) {
  __shared__ Smem sm;
  const int E = args.group_ends ? args.E : 1;
  const int32_t M = args.M;
  // tiles per group (order[] reused as scratch for the counts)
  for (int g = threadIdx.x; g < E; g += kThreads) {
    int32_t b = 0, e = M;
    if (args.group_ends) group_range(args.group_ends, g, M, b, e);
    sm.order[g] = (e - b + kTileQ - 1) / kTileQ;
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
    const uint32_t q0 = (uint32_t)gb + (mt - (uint32_t)sm.sched[g]) * kTileQ;
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
      P.scale = make_rsrc(wsg, (uint32_t)((int64_t)(args.N - 1) * args.ldws + K / 32));
      P.lds = (uint32_t)args.ldws;
      Q.scale = make_rsrc(args.as, (uint32_t)((int64_t)(M - 1) * args.ldas + K / 32));
      Q.lds = (uint32_t)args.ldas;
    }
    v16f acc[4][4];
    // scale rows start 4-byte aligned when both row strides are multiples of 4
    const bool scale_aligned = (args.ldas % 4 == 0) && (args.ldws % 4 == 0);
    mainloop<SCALED>(sm, P, Q, 0u, K, scale_aligned, acc);
    const int64_t ldo_bytes = args.ldo * (F32 ? 4 : 2);
    epilogue<F32>(acc, reinterpret_cast<char*>(args.out), ldo_bytes, q0, (uint32_t)ge, p0,
                  (uint32_t)args.N);
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
      P.scale = make_rsrc(args.ias, (uint32_t)((int64_t)(args.K - 1) * args.ldias + M / 32));
      P.lds = (uint32_t)args.ldias;
      Q.scale = make_rsrc(args.gos, (uint32_t)((int64_t)(args.N - 1) * args.ldgos + M / 32));
      Q.lds = (uint32_t)args.ldgos;
    }
    v16f acc[4][4];
    const bool scale_aligned =
        (args.ldias % 4 == 0) && (args.ldgos % 4 == 0) && ((tb >> 5) % 4 == 0);
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
      mainloop<SCALED>(sm, P, Q, (uint32_t)tb, (uint32_t)te, scale_aligned, acc);
    }
    char* out = reinterpret_cast<char*>(args.dw) +
                (int64_t)g * args.N * args.K * (F32 ? 4 : 2);
    epilogue<F32>(acc, out, (int64_t)args.K * (F32 ? 4 : 2), q0, (uint32_t)args.N, p0,
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
