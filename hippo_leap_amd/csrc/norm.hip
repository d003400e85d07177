// RMSNorm of the hidden state around the attention block, fp32 on the
// reference's column-major activations:
//   * rmsnorm_cols_kernel: gpuRmsnormCols (backends/naive.nim:2801-2843),
//     the norm in front of the Q/K/V projections (naive.nim:4063, 4095) and
//     the final norm before the logits (naive.nim:5537):
//     out[r, t] = x[r, t] * (1/sqrtf(sum_r x[r, t]^2 / dim + eps)) * w[r].
//   * residual_rmsnorm_kernel: gpuResidualRmsnorm (naive.nim:2845-2882), the
//     end of a decode layer (naive.nim:5530): x += residual in place, then
//     out = rmsnorm(x) * w.
//   * norm_vec4_kernel: both, for one aligned vector of dim % 4 == 0 (the
//     decode step), in one 1024-thread workgroup with the vector in registers.
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

// x = xin + res (xin may be x), out = rmsnorm(x) * w (out may be xin: each
// thread reads its own elements of xin before the barrier and writes them
// after it).
__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(float* x, const float* xin,
                                                               const float* __restrict__ res,
                                                               const float* __restrict__ w,
                                                               float* out, int dim, float eps) {
  float ss = 0.f;
  for (int r = threadIdx.x; r < dim; r += 256) {
    const float v = xin[r] + res[r];
    x[r] = v;
    ss += v * v;
  }
  const float inv = 1.0f / sqrtf(block_sum(ss) / (float)dim + eps);
  for (int r = threadIdx.x; r < dim; r += 256) out[r] = x[r] * inv * w[r];
}

// dim % 4 == 0, 16-byte aligned vectors, dim <= 16384: 1024 threads, up to
// four float4 chunks each, all loaded before the reduction and kept in
// registers for the second pass (the scalar loop above runs ~16 dependent
// load/store rounds per thread at dim 4096).  The weights are loaded with x,
// so the kernel waits for memory once.
// RES: x = xin + res first (xin may be x; out may be xin, as above).
template <bool RES>
__global__ __launch_bounds__(1024) void norm_vec4_kernel(float* x, const float* xin,
                                                         const float* __restrict__ res,
                                                         const float* __restrict__ w,
                                                         float* out, int dim, float eps) {
  __shared__ float part[16];
  const int n4 = dim >> 2, tid = threadIdx.x;
  f32x4 v[4], wv[4];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = tid + 1024 * k;
    v[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    wv[k] = v[k];
    if (c < n4) {
      v[k] = ((const f32x4*)xin)[c];
      if (RES) v[k] += ((const f32x4*)res)[c];
      wv[k] = ((const f32x4*)w)[c];
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = tid + 1024 * k;
    if (c < n4) {
      if (RES) ((f32x4*)x)[c] = v[k];
      ss += (v[k].x * v[k].x + v[k].y * v[k].y) + (v[k].z * v[k].z + v[k].w * v[k].w);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) t += part[i];
  const float inv = 1.0f / sqrtf(t / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = tid + 1024 * k;
    if (c < n4)
      ((f32x4*)out)[c] = f32x4{v[k].x * inv * wv[k].x, v[k].y * inv * wv[k].y,
                               v[k].z * inv * wv[k].z, v[k].w * inv * wv[k].w};
  }
}

bool vec4_ok(int dim, const void* a, const void* b, const void* c, const void* d) {
  const uintptr_t m = (uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)d;
  return dim % 4 == 0 && dim <= 16384 && (m & 15) == 0;
}

}  // namespace

hipError_t rmsnorm_cols_launch(float* out, const float* x, const float* w, int dim, int seq,
                               float eps, hipStream_t stream) {
  if (seq == 1 && vec4_ok(dim, x, w, out, out))
    hipLaunchKernelGGL(norm_vec4_kernel<false>, dim3(1), dim3(1024), 0, stream, const_cast<float*>(x), x,
                       nullptr, w, out, dim, eps);
  else if (seq < 64)
    hipLaunchKernelGGL(rmsnorm_col_kernel, dim3(seq), dim3(256), 0, stream, x, w, out, dim, seq, eps);
  else
    hipLaunchKernelGGL(rmsnorm_cols64_kernel, dim3((seq + 63) / 64), dim3(256), 0, stream, x, w,
                       out, dim, seq, eps);
  return hipGetLastError();
}

hipError_t residual_rmsnorm_from_launch(float* out, float* x_dst, const float* x_in, const float* res,
                                        const float* w, int dim, float eps, hipStream_t stream) {
  if (vec4_ok(dim, x_dst, res, w, out) && ((uintptr_t)x_in & 15) == 0)
    hipLaunchKernelGGL(norm_vec4_kernel<true>, dim3(1), dim3(1024), 0, stream, x_dst, x_in, res, w, out, dim, eps);
  else
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(1), dim3(256), 0, stream, x_dst, x_in, res, w, out, dim,
                       eps);
  return hipGetLastError();
}

hipError_t residual_rmsnorm_launch(float* out, float* x, const float* res, const float* w, int dim,
                                   float eps, hipStream_t stream) {
  return residual_rmsnorm_from_launch(out, x, x, res, w, dim, eps, stream);
}

}  // namespace hl
