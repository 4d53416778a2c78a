// Token routing around the expert GEMMs of a top-k MoE layer on one GPU.
//
// Dispatch plan: the (token, k) slots s = t * topk + k are sorted by expert,
// stably (slots of one expert keep their slot order), and each expert's run
// of rows is padded with empty rows to a multiple of `pad`.  Outputs:
//   perm[s]  row of slot s in the expert-ordered layout (-1: expert id out of
//            range, the slot is dropped)
//   src[r]   slot held by row r (-1: padding, including every row past the
//            last expert up to the capacity)
//   ends[e]  cumulative padded row ends (the group ends of the GEMMs)
//   counts[e] slots routed to expert e
// The reference's trainer gets this from torchtitan's token dispatcher with
// pad_multiple = 32 (port_mxfp8.py:214, 240), which sorts slots with a stable
// argsort of the expert ids; this is the same order.
//
// One form of the plan is one workgroup of 1024 threads (16 waves), so no
// grid-wide synchronisation and no host round trip are needed: each wave
// counts the experts of a contiguous slot range into its own LDS histogram,
// one thread per expert turns the histograms into per-wave starting rows, and
// each wave then walks its range again in 64-slot chunks, ranking equal
// experts inside a chunk with one ballot per key bit.  The other form runs the
// same steps over one workgroup per 4096 slots, with the per-workgroup counts
// in a caller's workspace and one small kernel between the two passes.
//
// Combine: out[t] = bf16(sum_k float(bf16(float(y[perm[s]]) * score[s]))),
// summed in fp32 in k order (the routed output scaled by its score and rounded
// to bf16 as the dispatcher does, then one rounding of the sum); without scores
// every term is the gathered row.  Its score gradient is the fp32 dot product
// of the output gradient with the gathered row.
#include <algorithm>

#include "mx_device.h"
#include "mxgg_internal.h"

namespace mxgg {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kPlanPrefetch = 8;  // 64-slot chunks whose ids are loaded together

// Lanes of the wave whose key equals this lane's (keys < 2^nbits).
__device__ __forceinline__ uint64_t match_key(uint32_t key, int nbits) {
  uint64_t m = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    const uint64_t ones = __ballot((key >> b) & 1u);
    m &= ((key >> b) & 1u) ? ones : ~ones;
  }
  return m;
}

// Counts the experts of slots [beg, end) of a wave into the LDS histogram h
// (ids outside [0, E) are not counted); the ids of kPlanPrefetch 64-slot
// chunks are loaded together, so that many loads are in flight.
__device__ __forceinline__ void count_range(const int32_t* __restrict__ idx, int64_t beg,
                                            int64_t end, int E, int32_t* h) {
  const int lane = threadIdx.x & 63;
  for (int64_t b0 = beg; b0 < end; b0 += 64 * kPlanPrefetch) {
    int32_t ev[kPlanPrefetch];
#pragma unroll
    for (int j = 0; j < kPlanPrefetch; ++j) {
      const int64_t s = b0 + 64 * j + lane;
      ev[j] = s < end ? idx[s] : -1;
    }
#pragma unroll
    for (int j = 0; j < kPlanPrefetch; ++j)
      if (ev[j] >= 0 && ev[j] < E) atomicAdd(&h[ev[j]], 1);
  }
}

// Ranks slots [beg, end) of a wave in slot order, 64 at a time: h[e] holds
// the next row of expert e for this wave and advances by the slots of e in
// each chunk, which are ranked among themselves with one ballot per key bit.
// Writes perm[s] (-1 for a dropped slot) and src[row].
__device__ __forceinline__ void rank_range(const int32_t* __restrict__ idx, int64_t beg,
                                           int64_t end, int E, int32_t* h, int64_t cap,
                                           int32_t* __restrict__ perm,
                                           int32_t* __restrict__ src) {
  const int lane = threadIdx.x & 63;
  // keys 0..E-1 are experts, E marks a dropped or absent slot
  const int nbits = 32 - __builtin_clz((unsigned)E);
  for (int64_t b0 = beg; b0 < end; b0 += 64 * kPlanPrefetch) {
    int32_t ev[kPlanPrefetch];
#pragma unroll
    for (int j = 0; j < kPlanPrefetch; ++j) {
      const int64_t s = b0 + 64 * j + lane;
      ev[j] = s < end ? idx[s] : -1;
    }
#pragma unroll
    for (int j = 0; j < kPlanPrefetch; ++j) {
      const int64_t s = b0 + 64 * j + lane;
      const bool active = s < end;
      const int32_t e = ev[j];
      const bool valid = active && e >= 0 && e < E;
      const uint32_t key = valid ? (uint32_t)e : (uint32_t)E;
      const uint64_t peers = match_key(key, nbits);
      const uint64_t below = (1ull << lane) - 1ull;
      const uint64_t upto = (2ull << lane) - 1ull;  // lane 63: all lanes
      if (valid) {
        const int32_t base = h[e];
        const int32_t dest = base + __popcll(peers & below);
        perm[s] = dest;
        if (dest < cap) src[dest] = (int32_t)s;  // always true: dest < group end <= cap
        if ((peers & ~upto) == 0) h[e] = base + __popcll(peers);  // last lane of the group
      } else if (active) {
        perm[s] = -1;
      }
    }
  }
}

// Per expert, from the slot counts of the nv consecutive histograms
// hist[v * E + e]: each histogram's first row (exclusive prefix plus the
// expert's padded start), the group ends, the counts, and -1 in src for the
// padding rows and every row past the last group up to cap.  One workgroup of
// kPlanThreads >= E threads; every thread calls it.
__device__ void plan_offsets(int32_t* hist, int nv, int E, int pad, int64_t cap,
                             int32_t* __restrict__ src, int32_t* __restrict__ ends,
                             int32_t* __restrict__ counts, int32_t* scan, int32_t* total_s) {
  const int tid = threadIdx.x;
  int32_t cnt = 0, padded = 0;
  if (tid < E) {
    // the expert's total first: loads only, 8 in flight (the workspace form
    // reads them from global memory)
    for (int v0 = 0; v0 < nv; v0 += 8) {
      int32_t c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = v0 + j < nv ? hist[(int64_t)(v0 + j) * E + tid] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) cnt += c[j];
    }
    padded = (cnt + pad - 1) / pad * pad;
  }
  // exclusive scan of the padded sizes over experts
  scan[tid] = padded;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const int32_t add = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += add;
    __syncthreads();
  }
  const int32_t start = scan[tid] - padded;
  if (tid < E) {
    ends[tid] = scan[tid];
    counts[tid] = cnt;
    // each histogram's first row: the expert's start plus the counts before
    // it (8 loads issued before their 8 stores)
    int32_t row = start;
    for (int v0 = 0; v0 < nv; v0 += 8) {
      int32_t c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = v0 + j < nv ? hist[(int64_t)(v0 + j) * E + tid] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (v0 + j < nv) hist[(int64_t)(v0 + j) * E + tid] = row;
        row += c[j];
      }
    }
    for (int32_t r = start + cnt; r < start + padded; ++r) src[r] = -1;
  }
  if (tid == E - 1) *total_s = scan[tid];
  __syncthreads();
  for (int64_t r = (int64_t)*total_s + tid; r < cap; r += kPlanThreads) src[r] = -1;
}

__global__ __launch_bounds__(kPlanThreads) void k_route_plan(
    const int32_t* __restrict__ idx, int64_t n, int E, int pad, int64_t cap,
    int32_t* __restrict__ perm, int32_t* __restrict__ src, int32_t* __restrict__ ends,
    int32_t* __restrict__ counts) {
  __shared__ int32_t hist[kPlanWaves * kMaxGroups];  // [wave][expert]
  __shared__ int32_t scan[kPlanThreads];
  __shared__ int32_t total_s;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  for (int i = tid; i < kPlanWaves * E; i += kPlanThreads) hist[i] = 0;
  __syncthreads();
  // Slot range of wave w: [beg, end), chunk-aligned.
  const int64_t per = ((n + kPlanWaves - 1) / kPlanWaves + 63) / 64 * 64;
  const int64_t beg = std::min<int64_t>((int64_t)w * per, n);
  const int64_t end = std::min<int64_t>(beg + per, n);
  count_range(idx, beg, end, E, hist + w * E);
  __syncthreads();
  plan_offsets(hist, kPlanWaves, E, pad, cap, src, ends, counts, scan, &total_s);
  rank_range(idx, beg, end, E, hist + w * E, cap, perm, src);
}

// The same plan over many workgroups, for the stores of routings past a few
// thousand slots (one workgroup writes perm and src at one CU's store rate):
// block b of the grid owns slots [b * kPlanBlockSlots, ...).
//   k_plan_count : the block's expert counts into ws[b][e] (global memory);
//   k_plan_offsets (one workgroup): ws[b][e] becomes the block's first row of
//                  expert e; group ends, counts and the -1 rows of src;
//   k_plan_rank  : the block's waves count their quarter-ranges again, take
//                  their first rows from ws[b][*] plus the waves before them,
//                  and rank as the one-workgroup plan does.
// The result is the one-workgroup plan's, bit for bit: both are the stable
// order by expert, which is unique.
constexpr int kPlanBlockThreads = 512;
constexpr int kPlanBlockWaves = kPlanBlockThreads / 64;
constexpr int64_t kPlanBlockSlots = 4096;

__global__ __launch_bounds__(kPlanBlockThreads) void k_plan_count(
    const int32_t* __restrict__ idx, int64_t n, int E, int32_t* __restrict__ ws) {
  __shared__ int32_t hist[kMaxGroups];
  const int tid = threadIdx.x;
  for (int i = tid; i < E; i += kPlanBlockThreads) hist[i] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * kPlanBlockSlots;
  const int64_t hi = std::min<int64_t>(lo + kPlanBlockSlots, n);
  const int64_t per = kPlanBlockSlots / kPlanBlockWaves;
  const int64_t beg = std::min<int64_t>(lo + (int64_t)(tid >> 6) * per, hi);
  count_range(idx, beg, std::min<int64_t>(beg + per, hi), E, hist);
  __syncthreads();
  for (int i = tid; i < E; i += kPlanBlockThreads) ws[(int64_t)blockIdx.x * E + i] = hist[i];
}

__global__ __launch_bounds__(kPlanThreads) void k_plan_offsets(
    int32_t* __restrict__ ws, int nblocks, int E, int pad, int64_t cap,
    int32_t* __restrict__ src, int32_t* __restrict__ ends, int32_t* __restrict__ counts) {
  __shared__ int32_t scan[kPlanThreads];
  __shared__ int32_t total_s;
  plan_offsets(ws, nblocks, E, pad, cap, src, ends, counts, scan, &total_s);
}

__global__ __launch_bounds__(kPlanBlockThreads) void k_plan_rank(
    const int32_t* __restrict__ idx, int64_t n, int E, int64_t cap,
    const int32_t* __restrict__ ws, int32_t* __restrict__ perm, int32_t* __restrict__ src) {
  __shared__ int32_t hist[kPlanBlockWaves * kMaxGroups];  // [wave][expert]
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  for (int i = tid; i < kPlanBlockWaves * E; i += kPlanBlockThreads) hist[i] = 0;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * kPlanBlockSlots;
  const int64_t hi = std::min<int64_t>(lo + kPlanBlockSlots, n);
  const int64_t per = kPlanBlockSlots / kPlanBlockWaves;
  const int64_t beg = std::min<int64_t>(lo + (int64_t)w * per, hi);
  const int64_t end = std::min<int64_t>(beg + per, hi);
  count_range(idx, beg, end, E, hist + w * E);
  __syncthreads();
  for (int e = tid; e < E; e += kPlanBlockThreads) {
    int32_t row = ws[(int64_t)blockIdx.x * E + e];
    for (int v = 0; v < kPlanBlockWaves; ++v) {
      const int32_t c = hist[v * E + e];
      hist[v * E + e] = row;
      row += c;
    }
  }
  __syncthreads();
  rank_range(idx, beg, end, E, hist + w * E, cap, perm, src);
}

// One wave per output row; lane l handles the 16-byte chunks l, l + 64, ...
// out[r] = x[src[r] / topk] (times row_scale[src[r]] when given); zero for
// src < 0 and for a slot whose token is not below xrows.
__global__ __launch_bounds__(256) void k_gather_rows(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t xrows, const int32_t* __restrict__ src,
    int topk, const float* __restrict__ row_scale, int64_t rows, int chunks,
    uint16_t* __restrict__ out, int64_t ldo) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int32_t sl = src[r];
  const bool ok = sl >= 0 && sl / topk < xrows;
  const uint16_t* xr = ok ? x + (int64_t)(sl / topk) * ldx : nullptr;
  const float sc = (ok && row_scale != nullptr) ? row_scale[sl] : 1.0f;
  uint16_t* o = out + r * ldo;
  for (int c = lane; c < chunks; c += 64) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (xr != nullptr) {
      v = *reinterpret_cast<const uint4*>(xr + 8 * c);
      if (row_scale != nullptr) v = scale_chunk(v, sc);
    }
    *reinterpret_cast<uint4*>(o + 8 * c) = v;
  }
}

// One wave per token.  out[t] = bf16(sum_k term_k), term_k =
// float(bf16(float(y[perm[s]]) * score[s])) (or the row itself without scores).
// Up to 8 slots per token: the slots' rows and factors are read once (they
// are the same for the whole wave) and every chunk's 8 row loads go out
// together; the sum stays in k order.  More slots take the general loop.
constexpr int kCombineSlots = 8;
constexpr int kCombineChunks = 4;

template <bool SCORES>
__global__ __launch_bounds__(256) void k_combine(
    const uint16_t* __restrict__ y, int64_t ldy, int64_t yrows, const int32_t* __restrict__ perm,
    const float* __restrict__ scores, int64_t tokens, int topk, int chunks,
    uint16_t* __restrict__ out, int64_t ldo) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (t >= tokens) return;
  const int32_t* pt = perm + t * topk;
  uint16_t* o = out + t * ldo;
  if (topk <= kCombineSlots) {
    int32_t r[kCombineSlots];
    float sc[kCombineSlots];
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) {
      const int32_t rk = k < topk ? pt[k] : -1;
      r[k] = rk >= 0 && rk < yrows ? rk : -1;
      sc[k] = SCORES && k < topk ? scores[t * topk + k] : 1.0f;
    }
    // kCombineChunks chunks of every slot row per trip: their 32 loads go out
    // together (C5: 430 -> 416 us against one chunk per trip)
    for (int c0 = lane; c0 < chunks; c0 += 64 * kCombineChunks) {
      uint4 v[kCombineChunks][kCombineSlots];
#pragma unroll
      for (int u = 0; u < kCombineChunks; ++u) {
        const int c = c0 + 64 * u;
#pragma unroll
        for (int k = 0; k < kCombineSlots; ++k)
          v[u][k] = r[k] >= 0 && c < chunks
                        ? *reinterpret_cast<const uint4*>(y + (int64_t)r[k] * ldy + 8 * c)
                        : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kCombineChunks; ++u) {
        const int c = c0 + 64 * u;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll
        for (int k = 0; k < kCombineSlots; ++k) {
          if (r[k] < 0) continue;
          const uint4 w = SCORES ? scale_chunk(v[u][k], sc[k]) : v[u][k];
          acc[0] += bf16_lo(w.x); acc[1] += bf16_hi(w.x);
          acc[2] += bf16_lo(w.y); acc[3] += bf16_hi(w.y);
          acc[4] += bf16_lo(w.z); acc[5] += bf16_hi(w.z);
          acc[6] += bf16_lo(w.w); acc[7] += bf16_hi(w.w);
        }
        // the combined rows are not read again here: streaming store (+2%)
        if (c < chunks)
          __builtin_nontemporal_store(
              u32x4{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                    pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7])},
              reinterpret_cast<u32x4*>(o + 8 * c));
      }
    }
    return;
  }
  for (int c = lane; c < chunks; c += 64) {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int k = 0; k < topk; ++k) {
      const int32_t r = pt[k];
      if (r < 0 || r >= yrows) continue;
      uint4 v = *reinterpret_cast<const uint4*>(y + (int64_t)r * ldy + 8 * c);
      if (SCORES) v = scale_chunk(v, scores[t * topk + k]);
      acc[0] += bf16_lo(v.x); acc[1] += bf16_hi(v.x);
      acc[2] += bf16_lo(v.y); acc[3] += bf16_hi(v.y);
      acc[4] += bf16_lo(v.z); acc[5] += bf16_hi(v.z);
      acc[6] += bf16_lo(v.w); acc[7] += bf16_hi(v.w);
    }
    *reinterpret_cast<uint4*>(o + 8 * c) =
        make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                   pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7]));
  }
}

__device__ __forceinline__ float dot_chunk(const uint4& d, const uint4& v, float acc) {
  acc = __builtin_fmaf(bf16_lo(d.x), bf16_lo(v.x), acc);
  acc = __builtin_fmaf(bf16_hi(d.x), bf16_hi(v.x), acc);
  acc = __builtin_fmaf(bf16_lo(d.y), bf16_lo(v.y), acc);
  acc = __builtin_fmaf(bf16_hi(d.y), bf16_hi(v.y), acc);
  acc = __builtin_fmaf(bf16_lo(d.z), bf16_lo(v.z), acc);
  acc = __builtin_fmaf(bf16_hi(d.z), bf16_hi(v.z), acc);
  acc = __builtin_fmaf(bf16_lo(d.w), bf16_lo(v.w), acc);
  return __builtin_fmaf(bf16_hi(d.w), bf16_hi(v.w), acc);
}

// One wave per token: d_score[s] = sum_h float(dout[t][h]) * float(y[perm[s]][h]),
// 0 for a dropped slot.  Up to 8 slots per token share one read of dout.
__global__ __launch_bounds__(256) void k_combine_score_grad(
    const uint16_t* __restrict__ dout, int64_t ldd, const uint16_t* __restrict__ y, int64_t ldy,
    int64_t yrows, const int32_t* __restrict__ perm, int64_t tokens, int topk, int chunks,
    float* __restrict__ dscore) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (t >= tokens) return;
  const uint16_t* dr = dout + t * ldd;
  for (int k0 = 0; k0 < topk; k0 += kCombineSlots) {
    int32_t r[kCombineSlots];
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) {
      const int32_t rk = k0 + k < topk ? perm[t * topk + k0 + k] : -1;
      r[k] = rk >= 0 && rk < yrows ? rk : -1;
    }
    float acc[kCombineSlots];
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) acc[k] = 0.0f;
    for (int c = lane; c < chunks; c += 64) {
      const uint4 d = *reinterpret_cast<const uint4*>(dr + 8 * c);
      uint4 v[kCombineSlots];
#pragma unroll
      for (int k = 0; k < kCombineSlots; ++k)
        v[k] = r[k] >= 0 ? *reinterpret_cast<const uint4*>(y + (int64_t)r[k] * ldy + 8 * c)
                         : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < kCombineSlots; ++k) acc[k] = dot_chunk(d, v[k], acc[k]);
    }
#pragma unroll
    for (int k = 0; k < kCombineSlots; ++k) {
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) acc[k] += __shfl_xor(acc[k], off);
      if (lane == 0 && k0 + k < topk) dscore[t * topk + k0 + k] = r[k] >= 0 ? acc[k] : 0.0f;
    }
  }
}

}  // namespace

hipError_t launch_route_plan(const int32_t* idx, int64_t n, int E, int pad, int64_t cap,
                             int32_t* perm, int32_t* src, int32_t* ends, int32_t* counts,
                             hipStream_t stream) {
  hipLaunchKernelGGL(k_route_plan, dim3(1), dim3(kPlanThreads), 0, stream, idx, n, E, pad, cap,
                     perm, src, ends, counts);
  return hipGetLastError();
}

int64_t route_plan_blocks(int64_t n) { return (n + kPlanBlockSlots - 1) / kPlanBlockSlots; }

hipError_t launch_route_plan_blocks(const int32_t* idx, int64_t n, int E, int pad, int64_t cap,
                                    int32_t* perm, int32_t* src, int32_t* ends, int32_t* counts,
                                    int32_t* ws, hipStream_t stream) {
  const int64_t nb = route_plan_blocks(n);
  if (nb > 0) {
    hipLaunchKernelGGL(k_plan_count, dim3((unsigned)nb), dim3(kPlanBlockThreads), 0, stream, idx,
                       n, E, ws);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(k_plan_offsets, dim3(1), dim3(kPlanThreads), 0, stream, ws, (int)nb, E, pad,
                     cap, src, ends, counts);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || nb == 0) return err;
  hipLaunchKernelGGL(k_plan_rank, dim3((unsigned)nb), dim3(kPlanBlockThreads), 0, stream, idx, n,
                     E, cap, ws, perm, src);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const uint16_t* x, int64_t ldx, int64_t xrows, const int32_t* src,
                              int topk, const float* row_scale, int64_t rows, int64_t cols,
                              uint16_t* out, int64_t ldo, hipStream_t stream) {
  if (rows == 0 || cols == 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, ldx,
                     xrows, src, topk, row_scale, rows, (int)(cols / 8), out, ldo);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t* y, int64_t ldy, int64_t yrows, const int32_t* perm,
                          const float* scores, int64_t tokens, int topk, int64_t cols, uint16_t* out,
                          int64_t ldo, hipStream_t stream) {
  if (tokens == 0 || cols == 0) return hipSuccess;
  const dim3 grid((unsigned)((tokens + 3) / 4));
  if (scores != nullptr)
    hipLaunchKernelGGL((k_combine<true>), grid, dim3(256), 0, stream, y, ldy, yrows, perm, scores,
                       tokens, topk, (int)(cols / 8), out, ldo);
  else
    hipLaunchKernelGGL((k_combine<false>), grid, dim3(256), 0, stream, y, ldy, yrows, perm, scores,
                       tokens, topk, (int)(cols / 8), out, ldo);
  return hipGetLastError();
}

hipError_t launch_combine_score_grad(const uint16_t* dout, int64_t ldd, const uint16_t* y,
                                     int64_t ldy, int64_t yrows, const int32_t* perm,
                                     int64_t tokens, int topk, int64_t cols, float* dscore,
                                     hipStream_t stream) {
  if (tokens == 0) return hipSuccess;
  hipLaunchKernelGGL(k_combine_score_grad, dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0,
                     stream, dout, ldd, y, ldy, yrows, perm, tokens, topk, (int)(cols / 8), dscore);
  return hipGetLastError();
}

}  // namespace mxgg
