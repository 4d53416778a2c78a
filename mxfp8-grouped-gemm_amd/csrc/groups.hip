// Group-offset utilities around the grouped GEMMs (gfx950).
//
//   k_offs_to_ends : the reference's wgrad entry points document `offs` as
//                    per-expert group sizes (wgrad_fused.py:37), its wgrad
//                    benchmark passes sizes (bench_wgrad_dsv3.py:52) and its
//                    layer step passes cumulative ends (e2e_bench.py:42,117).
//                    One workgroup turns either form into the cumulative ends
//                    the kernels read, on the device (no host sync).
//   k_zero_tail    : rows past the last group end are written by no GEMM;
//                    callers that hand a whole [rows, cols] tensor to autograd
//                    zero them with this.
#include "mxgg_internal.h"

namespace mxgg {
namespace {

constexpr int kScanThreads = 1024;  // one thread per group (at most 1024 groups)

__global__ __launch_bounds__(kScanThreads) void k_offs_to_ends(const int32_t* __restrict__ offs,
                                                               int E, int64_t tokens, int kind,
                                                               int32_t* __restrict__ ends) {
  __shared__ int64_t scan[kScanThreads];
  const int t = threadIdx.x;
  const int32_t v = t < E ? offs[t] : 0;
  scan[t] = v;
  __syncthreads();
  for (int off = 1; off < kScanThreads; off <<= 1) {
    const int64_t add = t >= off ? scan[t - off] : 0;
    __syncthreads();
    scan[t] += add;
    __syncthreads();
  }
  // kind 2 (auto): sizes when they add up to exactly `tokens` and the last
  // entry alone does not (an ends vector covering every token ends at
  // `tokens`); otherwise cumulative ends.
  const int64_t total = scan[E - 1];
  const int32_t last = offs[E - 1];
  const bool sizes = kind == MXGG_OFFS_SIZES ||
                     (kind == MXGG_OFFS_AUTO && total == tokens && (int64_t)last < tokens);
  if (t < E) {
    const int64_t c = scan[t];
    ends[t] = sizes ? (int32_t)(c > INT32_MAX ? INT32_MAX : (c < INT32_MIN ? INT32_MIN : c)) : v;
  }
}

// Rows [last, rows) of out, last = the largest group end clamped to [0, rows]
// (the end of the last group under the monotone rule), set to zero in 16-byte
// pieces.  Grid-stride; every workgroup finds `last` itself.
__global__ __launch_bounds__(256) void k_zero_tail(uint8_t* __restrict__ out, int64_t rows,
                                                   int64_t chunks_per_row, int64_t ld_bytes,
                                                   const int32_t* __restrict__ ends, int E) {
  __shared__ int32_t red[256];
  int32_t m = 0;
  for (int g = threadIdx.x; g < E; g += 256) m = max(m, ends[g]);
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  const int64_t last = red[0] > rows ? rows : red[0];
  const int64_t work = (rows - last) * chunks_per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < work;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = last + i / chunks_per_row, c = i % chunks_per_row;
    *reinterpret_cast<uint4*>(out + r * ld_bytes + c * 16) = make_uint4(0, 0, 0, 0);
  }
}

}  // namespace

hipError_t launch_offs_to_ends(const int32_t* offs, int64_t E, int64_t tokens, int kind,
                               int32_t* ends, hipStream_t stream) {
  hipLaunchKernelGGL(k_offs_to_ends, dim3(1), dim3(kScanThreads), 0, stream, offs, (int)E, tokens,
                     kind, ends);
  return hipGetLastError();
}

hipError_t launch_zero_tail(uint8_t* out, int64_t rows, int64_t row_bytes, int64_t ld_bytes,
                            const int32_t* ends, int64_t E, hipStream_t stream) {
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  hipLaunchKernelGGL(k_zero_tail, dim3(2 * cus), dim3(256), 0, stream, out, rows, row_bytes / 16,
                     ld_bytes, ends, (int)E);
  return hipGetLastError();
}

}  // namespace mxgg
