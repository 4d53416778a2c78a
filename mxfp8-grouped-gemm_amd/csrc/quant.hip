// bf16 -> MXFP8 (e4m3 payload + E8M0 1x32 block scale) casts for gfx950.
//
// Both kernels are HBM-bound streaming kernels: every input byte is read once
// and every output byte written once, with 16-byte vector accesses.
//   dim0 : blocks along the contiguous dimension (forward operands, K-blocks).
//   dim1 : blocks along the row (token) dimension, restarting at every group
//          boundary, written transposed and zero-padded per group to a
//          multiple of 32 tokens (wgrad operands).
#include "mx_device.h"
#include "mxgg_internal.h"

namespace mxgg {
namespace {

// ---------------------------------------------------------------------------
// dim0.  A wave covers 64 chunks of 8 bf16 (16 B) of one row; the four lanes
// of a quad hold one 32-element block and combine their amax with two DPP
// quad permutations.  Each wave loads 8 rows at once (a block 32 rows), so a
// quad ends a trip holding 8 scale bytes of one block column: with block-major
// scales those leave in one 8-byte store instead of eight byte stores.
// Payload stores are nontemporal.  (Measured on C2's X, 65536 x 7168:
// 4.8 TB/s with 4 rows per wave and byte scale stores, 5.7 TB/s so.)
// ---------------------------------------------------------------------------
// GATHER (1, or 2 with row factors): row r of the cast's input is row
// src[r] / topk of x (zero when src[r] < 0 or that token is not below xrows),
// with GATHER 2 times scale[src[r]] rounded to bf16: the routed layout of a
// top-k MoE layer read straight from token order (the dispatch's gather, or
// the combine's backward).  Separate instantiations keep the plain gather's
// registers free of the factors.
struct Gather {
  const int32_t* src;
  const float* scale;
  int64_t xrows;
  int topk;
};

// GATHER: the rows are gathered from token order as in k_quant_dim1 (no row
// factors): the row-wise cast of the routed layout for a forward-only pass.
template <int MODE, bool SW, bool GATHER>
__global__ __launch_bounds__(256) void k_quant_dim0(const uint16_t* __restrict__ x, int64_t rows,
                                                    int cols8, int64_t ldx,
                                                    uint8_t* __restrict__ q, int64_t ldq,
                                                    uint8_t* __restrict__ s, int64_t s_row,
                                                    int64_t s_blk, Gather ga) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // column blocks vary fastest over the grid for token-order rows, row blocks
  // for gathered rows (measured 7% faster at C5's routing)
  const uint32_t cb = GATHER ? blockIdx.y : blockIdx.x, rb = GATHER ? blockIdx.x : blockIdx.y;
  const uint32_t nrb = GATHER ? gridDim.x : gridDim.y;
  const int cc = cb * 64 + lane;          // chunk column
  const bool col_ok = cc < cols8;         // whole quads share col_ok (cols8 % 4 == 0)
  // block-major scales with 8-byte aligned block columns: one store per quad
  const bool pack_s = s_row == 1 && ((s_blk | (int64_t)(uintptr_t)s) & 7) == 0;
  for (int64_t r0 = (int64_t)rb * 32 + wave * 8; r0 < rows; r0 += (int64_t)nrb * 32) {
    uint4 v[8];
    if (GATHER) {
      int32_t sl[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) sl[u] = r0 + u < rows ? ga.src[r0 + u] : -1;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t t = sl[u] >= 0 ? sl[u] / ga.topk : ga.xrows;
        v[u] = col_ok && t < ga.xrows
                   ? *reinterpret_cast<const uint4*>(x + t * ldx + (int64_t)cc * 8)
                   : make_uint4(0, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t r = r0 + u;
        v[u] = col_ok && r < rows ? *reinterpret_cast<const uint4*>(x + r * ldx + (int64_t)cc * 8)
                                  : make_uint4(0, 0, 0, 0);
      }
    }
    uint32_t sw[2];  // scale bytes of rows r0 .. r0+7, packed
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t b[4];
      bool nan = false;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        b[u] = e8m0_from_amax16<MODE>(quad_max(amax16_of_chunk(v[4 * h + u])));
        nan |= needs_full_encoder<MODE, SW>(b[u]);
      }
      sw[h] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      const bool any_nan = __any(nan);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t r = r0 + 4 * h + u;
        const uint2 o = any_nan ? encode_chunk8<MODE, SW, true>(v[4 * h + u], b[u])
                                : encode_chunk8<MODE, SW, false>(v[4 * h + u], b[u]);
        if (col_ok && r < rows) store_stream(q + r * ldq + (int64_t)cc * 8, o);
      }
    }
    if ((lane & 3) == 0 && col_ok) {
      uint8_t* sp = s + (int64_t)(cc >> 2) * s_blk;
      if (pack_s && r0 + 8 <= rows) {
        *reinterpret_cast<uint2*>(sp + r0) = make_uint2(sw[0], sw[1]);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (r0 + u < rows) sp[(r0 + u) * s_row] = (uint8_t)(sw[u >> 2] >> (8 * (u & 3)));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Block-wide prefix over group sizes, kept in LDS.
//   ends_s[g]  : end of group g (unpadded; running maximum of the clamped ends)
//   pend_s[g]  : padded cumulative end (each group rounded up to 32 tokens)
// ---------------------------------------------------------------------------
__device__ void groups_to_lds(const int32_t* __restrict__ ends, int E, int64_t rows,
                              int32_t* ends_s, int32_t* pend_s, int32_t* tmp /*256*/) {
  const int t = threadIdx.x;
  monotone_ends_to_lds(ends, E, rows, ends_s);
  // Each thread owns up to 4 consecutive groups.
  int32_t local_pad[4];
  int32_t sum = 0;
  const int g0 = t * 4;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int g = g0 + u;
    int32_t pad = 0;
    if (g < E) {
      const int32_t sz = ends_s[g] - (g > 0 ? ends_s[g - 1] : 0);
      pad = (sz + 31) & ~31;
    }
    local_pad[u] = pad;
    sum += pad;
  }
  tmp[t] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int32_t add = t >= off ? tmp[t - off] : 0;
    __syncthreads();
    tmp[t] += add;
    __syncthreads();
  }
  int32_t run = t > 0 ? tmp[t - 1] : 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int g = g0 + u;
    run += local_pad[u];
    if (g < E) pend_s[g] = run;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Padded group ends for dim1 (one workgroup): ends_pad[g] = sum over groups
// <= g of round_up(size, 32), sizes taken from the monotone clamped ends.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pad_ends(const int32_t* __restrict__ ends, int E,
                                                  int64_t rows, int32_t* __restrict__ ends_pad) {
  __shared__ int32_t ends_s[kMaxGroups];
  __shared__ int32_t pend_s[kMaxGroups];
  __shared__ int32_t tmp[256];
  groups_to_lds(ends, E, rows, ends_s, pend_s, tmp);
  for (int g = threadIdx.x; g < E; g += 256) ends_pad[g] = pend_s[g];
}

// ---------------------------------------------------------------------------
// dim1.  A wave covers 128 padded token positions x 64 features; lane
// (fg = lane % 8, tg = lane / 8) owns positions 16*tg .. +15 of the tile and
// features 8*fg .. +7.  It loads its 16 token rows as 16-byte vectors (eight
// consecutive lanes read one whole 128-byte line of a row), takes each
// feature's amax over its 16 tokens (two features at once with packed 16-bit
// max), combines it with lane tg^1 = lane^8 (the other half of the 32-token
// block; a DPP rotation by 8 within the 16-lane row), and writes 16 payload
// bytes per feature (eight lanes write one whole 128-byte line of an output
// row).  No LDS transpose is needed.  Padded positions map to tokens through
// the padded group ends; a run of 16 never straddles two groups because every
// group starts on a multiple of 32.  A workgroup is 4 waves along the
// features (128 positions x 256 features).
//
// ROW (the dual cast) also writes the row-wise cast of the same data from the
// same registers: for each of its tokens a lane holds one 8-feature chunk, the
// quad fg = 4k .. 4k+3 holds a 32-feature block (amax over two DPP quad
// permutations, two tokens per step).  Every token inside a group is covered
// by exactly one lane run, so each row-wise row is written once.  (With the
// lanes the other way round, tg = lane % 8, the block took two LDS shuffles:
// the dual cast ran 3% and its gathered forms 12% slower.)
// ---------------------------------------------------------------------------
// Row-wise payload of a lane's 16 token chunks (row i at qrow + i * ldq).
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ void row_payload(const uint4 (&v)[16], const uint32_t (&rb)[16],
                                            uint8_t* qrow, int64_t ldq, int ntok) {
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < ntok)
      *reinterpret_cast<uint2*>(qrow + i * ldq) = encode_chunk8<MODE, SW, ANY>(v[i], rb[i]);
}

// Token-axis payload: feature j (half j & 1 of word j >> 1) of 16 positions,
// 16 bytes at row j of qrow.
template <int MODE, bool SW, bool ANY>
__device__ __forceinline__ void token_payload(const uint4 (&v)[16], const uint32_t (&bytes)[8],
                                              uint8_t* qrow, int64_t ldqt, bool out_ok) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = 4 * k + u;
        w[u] = (j >> 1) == 0 ? v[i].x : (j >> 1) == 1 ? v[i].y : (j >> 1) == 2 ? v[i].z : v[i].w;
      }
      // feature j of positions 4k .. 4k+3, paired into two bf16 words
      const uint32_t p0 = (j & 1) ? pair_halves<true>(w[0], w[1]) : pair_halves<false>(w[0], w[1]);
      const uint32_t p1 = (j & 1) ? pair_halves<true>(w[2], w[3]) : pair_halves<false>(w[2], w[3]);
      o[k] = encode4_words<MODE, SW, ANY>(p0, p1, bytes[j]);
    }
    // whole 128-byte lines (eight lanes): streaming stores (measured +1..4%;
    // the row-wise payload, 64-byte pieces of a line, is slower streamed)
    if (out_ok)
      __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]},
                                  reinterpret_cast<u32x4*>(qrow + (int64_t)j * ldqt));
  }
}

// Grid order of the token-axis cast (see k_quant_dim1).
template <int GATHER>
__host__ __device__ __forceinline__ bool feature_fastest(int64_t cap) {
  return GATHER == 0 && (cap + 127) / 128 <= 65535;
}

struct RowOut {
  uint8_t* q;     // [rows, cols] row-wise payload
  uint8_t* s;     // scale bytes, byte (r, b) at s[r * s_row + b * s_blk]
  int64_t ldq, s_row, s_blk;
};

// The gathered instantiations are capped at 128 VGPRs (four waves per SIMD,
// no spills): the extra wave hides the row-index load in front of every
// gathered row (measured +3% plain, +6% with row factors at C5's routing).
// The other instantiations keep their registers: capped, the dual cast of
// token-order rows ran 1% slower.
template <int MODE, bool SW, bool ROW, int GATHER>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GATHER ? 4 : 1))) void k_quant_dim1(
    const uint16_t* __restrict__ x, int64_t rows, int cols, int64_t ldx,
    const int32_t* __restrict__ ends, const int32_t* __restrict__ ends_pad, int E,
    int64_t rows_pad_cap, uint8_t* __restrict__ qt, int64_t ldqt, uint8_t* __restrict__ st,
    int64_t st_row, int64_t st_blk, RowOut ro, Gather ga) {
  __shared__ int32_t ends_s[kMaxGroups];
  __shared__ int32_t pend_s[kMaxGroups];
  const int lane = threadIdx.x & 63;
  const int fg = lane & 7, tg = lane >> 3;
  // Feature blocks vary fastest over the grid for token-order rows (the
  // workgroups reading the 256-feature pieces of the same 128 rows run
  // together: +8% on C4's dY, +4% dual), positions fastest for gathered rows
  // (measured 17% faster that way) and when the positions outgrow the grid's
  // y range (dim1_grid makes the same choice).
  const bool ffast = feature_fastest<GATHER>(rows_pad_cap);
  const uint32_t pblk = ffast ? blockIdx.y : blockIdx.x;
  const uint32_t fblk = ffast ? blockIdx.x : blockIdx.y;
  const int64_t P = (int64_t)pblk * 128 + 16 * tg;
  const int f = (int)fblk * 256 + (threadIdx.x >> 6) * 64 + 8 * fg;

  int64_t tok0 = 0;
  int ntok = 0;
  if (ends != nullptr) {
    stage_group_tables(ends, ends_pad, E, rows, ends_s, pend_s);
    __syncthreads();
    padded_run_tokens(P, 16, ends_s, pend_s, E, tok0, ntok);
  } else {
    tok0 = P;
    const int64_t n = rows - P;
    ntok = n <= 0 ? 0 : (n >= 16 ? 16 : (int)n);
  }
  if (f >= cols) ntok = 0;

  uint4 v[16];
  if (GATHER == 1) {
    // all 16 row indices first, then all 16 rows: two load latencies, not 16
    int32_t sl[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sl[i] = i < ntok ? ga.src[tok0 + i] : -1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t t = sl[i] >= 0 ? sl[i] / ga.topk : ga.xrows;
      v[i] = t < ga.xrows ? *reinterpret_cast<const uint4*>(x + t * ldx + f)
                          : make_uint4(0, 0, 0, 0);
    }
  } else if (GATHER == 2) {
    // the row factors are loaded together with the rows so that their
    // latency overlaps
    int32_t sl[16], t[16];
    float sc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sl[i] = i < ntok ? ga.src[tok0 + i] : -1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t ti = sl[i] >= 0 ? sl[i] / ga.topk : ga.xrows;
      t[i] = ti < ga.xrows ? (int32_t)ti : -1;
      sc[i] = t[i] >= 0 ? ga.scale[sl[i]] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[i] = t[i] >= 0 ? *reinterpret_cast<const uint4*>(x + (int64_t)t[i] * ldx + f)
                       : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (t[i] >= 0) v[i] = scale_chunk(v[i], sc[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[i] = i < ntok ? *reinterpret_cast<const uint4*>(x + (tok0 + i) * ldx + f)
                      : make_uint4(0, 0, 0, 0);
    }
  }

  if (ROW) {
    // Row-wise cast: block amax of token i in the low / high half of a word
    // for tokens 2t / 2t + 1, so one shuffle serves two tokens.
    uint32_t rb[16];
    bool nan = false;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // packed |x| maxima of the two chunks, then each chunk's two halves
      const uint32_t p0 = pk_max_u16(pk_max_u16(abs_bf16x2(v[2 * t].x), abs_bf16x2(v[2 * t].y)),
                                     pk_max_u16(abs_bf16x2(v[2 * t].z), abs_bf16x2(v[2 * t].w)));
      const uint32_t p1 =
          pk_max_u16(pk_max_u16(abs_bf16x2(v[2 * t + 1].x), abs_bf16x2(v[2 * t + 1].y)),
                     pk_max_u16(abs_bf16x2(v[2 * t + 1].z), abs_bf16x2(v[2 * t + 1].w)));
      uint32_t m = half_max_pair(p0, p1);
      m = pk_max_u16(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0xB1, 0xF, 0xF, false));
      m = pk_max_u16(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x4E, 0xF, 0xF, false));
      rb[2 * t] = e8m0_from_amax16<MODE>(m & 0xFFFFu);
      rb[2 * t + 1] = e8m0_from_amax16<MODE>(m >> 16);
      nan |= needs_full_encoder<MODE, SW>(rb[2 * t]) ||
             needs_full_encoder<MODE, SW>(rb[2 * t + 1]);
    }
    uint8_t* qrow = ro.q + tok0 * ro.ldq + f;
    if (__any(nan))
      row_payload<MODE, SW, true>(v, rb, qrow, ro.ldq, ntok);
    else
      row_payload<MODE, SW, false>(v, rb, qrow, ro.ldq, ntok);
    if ((fg & 3) == 0 && ntok > 0) {
      uint8_t* sp = ro.s + tok0 * ro.s_row + (int64_t)(f >> 5) * ro.s_blk;
      if (ro.s_row == 1 && ntok == 16) {
        store_scale_bytes16(sp, rb);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < ntok) sp[(int64_t)i * ro.s_row] = (uint8_t)rb[i];
      }
    }
  }

  if (ROW) __builtin_amdgcn_sched_barrier(0);  // keep the two casts' temporaries apart

  // Token-axis cast: features 2k, 2k + 1 are the halves of word k.
  const bool out_ok = f < cols && P < rows_pad_cap;
  uint32_t bytes[8];
  bool tnan = false;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t w = k == 0 ? v[i].x : k == 1 ? v[i].y : k == 2 ? v[i].z : v[i].w;
      m = pk_max_u16(m, abs_bf16x2(w));
    }
    m = pk_max_u16(m, (uint32_t)__builtin_amdgcn_update_dpp((int)m, (int)m, 0x128, 0xF, 0xF, false));
    bytes[2 * k] = e8m0_from_amax16<MODE>(m & 0xFFFFu);
    bytes[2 * k + 1] = e8m0_from_amax16<MODE>(m >> 16);
    tnan |= needs_full_encoder<MODE, SW>(bytes[2 * k]) ||
            needs_full_encoder<MODE, SW>(bytes[2 * k + 1]);
  }
  if (__any(tnan))
    token_payload<MODE, SW, true>(v, bytes, qt + (int64_t)f * ldqt + P, ldqt, out_ok);
  else
    token_payload<MODE, SW, false>(v, bytes, qt + (int64_t)f * ldqt + P, ldqt, out_ok);
  if (out_ok && (tg & 1) == 0) {
    uint8_t* sp = st + (int64_t)f * st_row + (P >> 5) * st_blk;
    if (st_row == 1 && (reinterpret_cast<uintptr_t>(sp) & 7u) == 0) {
      *reinterpret_cast<uint2*>(sp) = make_uint2(
          bytes[0] | (bytes[1] << 8) | (bytes[2] << 16) | (bytes[3] << 24),
          bytes[4] | (bytes[5] << 8) | (bytes[6] << 16) | (bytes[7] << 24));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) sp[(int64_t)j * st_row] = (uint8_t)bytes[j];
    }
  }
}

template <int MODE, bool SW, bool GATHER>
hipError_t dim0_impl(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx, uint8_t* q,
                     int64_t ldq, uint8_t* s, int64_t s_row, int64_t s_blk, const Gather& ga,
                     hipStream_t stream) {
  const int cols8 = (int)(cols / 8);
  const unsigned cblocks = (unsigned)((cols8 + 63) / 64);
  const dim3 grid = GATHER ? dim3((unsigned)std::min<int64_t>((rows + 31) / 32, 1 << 20), cblocks)
                           : dim3(cblocks, (unsigned)std::min<int64_t>((rows + 31) / 32, 65535));
  hipLaunchKernelGGL((k_quant_dim0<MODE, SW, GATHER>), grid, dim3(256), 0, stream, x, rows, cols8,
                     ldx, q, ldq, s, s_row, s_blk, ga);
  return hipGetLastError();
}

template <int MODE, bool SW, bool ROW, int GATHER>
hipError_t dim1_impl(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                     const int32_t* ends, int64_t E, int64_t cap, uint8_t* qt, int64_t ldqt,
                     uint8_t* st, int64_t st_row, int64_t st_blk, int32_t* ends_pad,
                     const RowOut& ro, const Gather& ga, hipStream_t stream) {
  if (ends != nullptr) {
    hipLaunchKernelGGL(k_pad_ends, dim3(1), dim3(256), 0, stream, ends, (int)E, rows, ends_pad);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  const unsigned pblocks = (unsigned)((cap + 127) / 128), fblocks = (unsigned)((cols + 255) / 256);
  const dim3 grid = feature_fastest<GATHER>(cap) ? dim3(fblocks, pblocks) : dim3(pblocks, fblocks);
  hipLaunchKernelGGL((k_quant_dim1<MODE, SW, ROW, GATHER>), grid, dim3(256), 0, stream, x, rows,
                     (int)cols, ldx, ends, ends_pad, (int)E, cap, qt, ldqt, st, st_row, st_blk, ro,
                     ga);
  return hipGetLastError();
}

// Row-major [batch][rows][nblk] E8M0 -> block-major [batch][nblk][rows]
// through a 64x64 LDS tile: coalesced reads along blocks, writes along rows.
__global__ __launch_bounds__(256) void k_scales_to_block_major(
    const uint8_t* __restrict__ src, int64_t rows, int64_t nblk, int64_t sb, int64_t lds,
    uint8_t* __restrict__ dst, int64_t db, int64_t ldd) {
  __shared__ uint8_t tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, k = k0 + tx;
    if (r < rows && k < nblk) tile[i][tx] = src[b * sb + r * lds + k];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t k = k0 + i, r = r0 + tx;
    if (r < rows && k < nblk) dst[b * db + k * ldd + r] = tile[tx][i];
  }
}

}  // namespace

template <bool GATHER>
hipError_t quant_dim0(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx, uint8_t* q,
                      int64_t ldq, uint8_t* s, int64_t lds, int layout, int mode,
                      const Gather& ga, hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const bool sw = (mode & kCvtSoftwareFlag) != 0;
  const int m = mode & 0xFF;
  const int64_t s_row = layout == MXGG_SCALES_BLOCK_MAJOR ? 1 : lds;
  const int64_t s_blk = layout == MXGG_SCALES_BLOCK_MAJOR ? lds : 1;
  if (m == kModeRceil)
    return sw ? dim0_impl<kModeRceil, true, GATHER>(x, rows, cols, ldx, q, ldq, s, s_row, s_blk,
                                                    ga, stream)
              : dim0_impl<kModeRceil, false, GATHER>(x, rows, cols, ldx, q, ldq, s, s_row, s_blk,
                                                     ga, stream);
  return sw ? dim0_impl<kModeFloor, true, GATHER>(x, rows, cols, ldx, q, ldq, s, s_row, s_blk,
                                                  ga, stream)
            : dim0_impl<kModeFloor, false, GATHER>(x, rows, cols, ldx, q, ldq, s, s_row, s_blk,
                                                   ga, stream);
}

hipError_t launch_quant_dim0(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                             uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, int layout,
                             int mode, hipStream_t stream) {
  return quant_dim0<false>(x, rows, cols, ldx, q, ldq, s, lds, layout, mode, Gather{}, stream);
}

hipError_t launch_gather_quant_dim0(const uint16_t* x, int64_t xrows, int64_t ldx,
                                    const int32_t* src, int topk, int64_t rows, int64_t cols,
                                    uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, int layout,
                                    int mode, hipStream_t stream) {
  Gather ga;
  ga.src = src;
  ga.scale = nullptr;
  ga.xrows = xrows;
  ga.topk = topk;
  return quant_dim0<true>(x, rows, cols, ldx, q, ldq, s, lds, layout, mode, ga, stream);
}

hipError_t launch_quant_dim1(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                             const int32_t* group_ends, int64_t num_groups,
                             int64_t rows_pad_cap, uint8_t* qt, int64_t ldqt, uint8_t* st,
                             int64_t ldst, int layout, int32_t* group_ends_pad, int mode,
                             hipStream_t stream) {
  return launch_quant_dual(x, rows, cols, ldx, group_ends, num_groups, rows_pad_cap, nullptr, 0,
                           nullptr, 0, qt, ldqt, st, ldst, layout, group_ends_pad, mode, stream);
}

template <int GATHER>
hipError_t quant_dual(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                      const int32_t* group_ends, int64_t num_groups, int64_t rows_pad_cap,
                      uint8_t* q, int64_t ldq, uint8_t* s, int64_t lds, uint8_t* qt, int64_t ldqt,
                      uint8_t* st, int64_t ldst, int layout, int32_t* group_ends_pad, int mode,
                      const Gather& ga, hipStream_t stream) {
  if (cols == 0 || rows_pad_cap == 0) return hipSuccess;
  const bool sw = (mode & kCvtSoftwareFlag) != 0;
  const int m = mode & 0xFF;
  const bool bm = layout == MXGG_SCALES_BLOCK_MAJOR;
  const int64_t st_row = bm ? 1 : ldst;
  const int64_t st_blk = bm ? ldst : 1;
  RowOut ro;
  ro.q = q;
  ro.s = s;
  ro.ldq = ldq;
  ro.s_row = bm ? 1 : lds;
  ro.s_blk = bm ? lds : 1;
#define MXGG_DIM1(MODE, SWF, ROWF)                                                           \
  dim1_impl<MODE, SWF, ROWF, GATHER>(x, rows, cols, ldx, group_ends, num_groups, rows_pad_cap, \
                                     qt, ldqt, st, st_row, st_blk, group_ends_pad, ro, ga, stream)
  if (q == nullptr) {
    if (m == kModeRceil)
      return sw ? MXGG_DIM1(kModeRceil, true, false) : MXGG_DIM1(kModeRceil, false, false);
    return sw ? MXGG_DIM1(kModeFloor, true, false) : MXGG_DIM1(kModeFloor, false, false);
  }
  if (m == kModeRceil)
    return sw ? MXGG_DIM1(kModeRceil, true, true) : MXGG_DIM1(kModeRceil, false, true);
  return sw ? MXGG_DIM1(kModeFloor, true, true) : MXGG_DIM1(kModeFloor, false, true);
#undef MXGG_DIM1
}

hipError_t launch_quant_dual(const uint16_t* x, int64_t rows, int64_t cols, int64_t ldx,
                             const int32_t* group_ends, int64_t num_groups,
                             int64_t rows_pad_cap, uint8_t* q, int64_t ldq, uint8_t* s,
                             int64_t lds, uint8_t* qt, int64_t ldqt, uint8_t* st, int64_t ldst,
                             int layout, int32_t* group_ends_pad, int mode, hipStream_t stream) {
  return quant_dual<0>(x, rows, cols, ldx, group_ends, num_groups, rows_pad_cap, q, ldq, s, lds,
                       qt, ldqt, st, ldst, layout, group_ends_pad, mode, Gather{}, stream);
}

hipError_t launch_gather_quant_dual(const uint16_t* x, int64_t xrows, int64_t ldx,
                                    const int32_t* src, int topk, const float* row_scale,
                                    int64_t rows, int64_t cols, const int32_t* group_ends,
                                    int64_t num_groups, int64_t rows_pad_cap, uint8_t* q,
                                    int64_t ldq, uint8_t* s, int64_t lds, uint8_t* qt,
                                    int64_t ldqt, uint8_t* st, int64_t ldst, int layout,
                                    int32_t* group_ends_pad, int mode, hipStream_t stream) {
  Gather ga;
  ga.src = src;
  ga.scale = row_scale;
  ga.xrows = xrows;
  ga.topk = topk;
  if (row_scale != nullptr)
    return quant_dual<2>(x, rows, cols, ldx, group_ends, num_groups, rows_pad_cap, q, ldq, s, lds,
                         qt, ldqt, st, ldst, layout, group_ends_pad, mode, ga, stream);
  return quant_dual<1>(x, rows, cols, ldx, group_ends, num_groups, rows_pad_cap, q, ldq, s, lds,
                       qt, ldqt, st, ldst, layout, group_ends_pad, mode, ga, stream);
}

hipError_t launch_pad_ends(const int32_t* group_ends, int64_t num_groups, int64_t rows,
                           int32_t* group_ends_pad, hipStream_t stream) {
  hipLaunchKernelGGL(k_pad_ends, dim3(1), dim3(256), 0, stream, group_ends, (int)num_groups, rows,
                     group_ends_pad);
  return hipGetLastError();
}

hipError_t launch_scales_to_block_major(const uint8_t* src, int64_t batch, int64_t rows,
                                        int64_t nblk, int64_t sb, int64_t lds, uint8_t* dst,
                                        int64_t db, int64_t ldd, hipStream_t stream) {
  if (batch == 0 || rows == 0 || nblk == 0) return hipSuccess;
  dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((nblk + 63) / 64), (unsigned)batch);
  hipLaunchKernelGGL(k_scales_to_block_major, grid, dim3(256), 0, stream, src, rows, nblk, sb, lds,
                     dst, db, ldd);
  return hipGetLastError();
}

}  // namespace mxgg
