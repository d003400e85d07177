// RMSNorm of the hidden state around the attention block, fp32 on the
// reference's column-major activations:
//   * rmsnorm_cols_kernel: gpuRmsnormCols (backends/naive.nim:2801-2843),
//     the norm in front of the Q/K/V projections (naive.nim:4063, 4095) and
//     the final norm before the logits (naive.nim:5537):
//     out[r, t] = x[r, t] * (1/sqrtf(sum_r x[r, t]^2 / dim + eps)) * w[r].
//   * residual_rmsnorm_kernel: gpuResidualRmsnorm (naive.nim:2845-2882), the
//     end of a decode layer (naive.nim:5530): x += residual in place, then
//     out = rmsnorm(x) * w.
// Both are HBM/latency-bound; sums of squares are fp32, reduced in a
// different order than the reference's 256-thread LDS tree.
#include "common.h"
#include "launch.h"

namespace hl {
namespace {

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// 256-thread sum (every thread gets the total).
__device__ inline float block_sum(float v) {
  __shared__ float part[4];
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return (part[0] + part[1]) + (part[2] + part[3]);
}

// One column (seq_len == 1, or one workgroup per column when seq_len is
// small): 256 threads stride over the rows.
__global__ __launch_bounds__(256) void rmsnorm_col_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          float* out, int dim, int seq, float eps) {
  const int col = blockIdx.x;
  float ss = 0.f;
  for (int r = threadIdx.x; r < dim; r += 256) {
    const float v = x[(size_t)r * seq + col];
    ss += v * v;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss) / (float)dim + eps);
  for (int r = threadIdx.x; r < dim; r += 256) {
    const size_t i = (size_t)r * seq + col;
    out[i] = x[i] * inv * w[r];
  }
}

// 64 adjacent columns per workgroup (lanes along t, coalesced), the four
// waves splitting the rows; the column sums meet in LDS.
__global__ __launch_bounds__(256) void rmsnorm_cols64_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ w,
                                                             float* out, int dim, int seq,
                                                             float eps) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  const bool live = col < seq;
  float ss = 0.f;
  if (live)
    for (int r = wave; r < dim; r += 4) {
      const float v = x[(size_t)r * seq + col];
      ss += v * v;
    }
  part[wave][lane] = ss;
  __syncthreads();
  const float tot = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
  const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
  if (live)
    for (int r = wave; r < dim; r += 4) {
      const size_t i = (size_t)r * seq + col;
      out[i] = x[i] * inv * w[r];
    }
}

__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(float* __restrict__ x,
                                                               const float* __restrict__ res,
                                                               const float* __restrict__ w,
                                                               float* __restrict__ out, int dim,
                                                               float eps) {
  float ss = 0.f;
  for (int r = threadIdx.x; r < dim; r += 256) {
    const float v = x[r] + res[r];
    x[r] = v;
    ss += v * v;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss) / (float)dim + eps);
  for (int r = threadIdx.x; r < dim; r += 256) out[r] = x[r] * inv * w[r];
}

}  // namespace

hipError_t rmsnorm_cols_launch(float* out, const float* x, const float* w, int dim, int seq,
                               float eps, hipStream_t stream) {
  if (seq < 64)
    hipLaunchKernelGGL(rmsnorm_col_kernel, dim3(seq), dim3(256), 0, stream, x, w, out, dim, seq, eps);
  else
    hipLaunchKernelGGL(rmsnorm_cols64_kernel, dim3((seq + 63) / 64), dim3(256), 0, stream, x, w,
                       out, dim, seq, eps);
  return hipGetLastError();
}

hipError_t residual_rmsnorm_launch(float* out, float* x, const float* res, const float* w, int dim,
                                   float eps, hipStream_t stream) {
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(1), dim3(256), 0, stream, x, res, w, out, dim, eps);
  return hipGetLastError();
}

}  // namespace hl
