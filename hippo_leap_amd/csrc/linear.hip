// fp32 linear layer over the reference's column-major activations: the
// drop-in for gpuLinearCol (backends/naive.nim:3519-3547), which the forward
// pass calls for the Q/K/V projections in front of attention and the O
// projection behind it (naive.nim:4064-4066, 4079).
//
//   Y[M, T] = W[M, K] . X[K, T]
//
// W is row-major with K fastest (the GGUF weight as loaded, naive.nim:4091);
// X and Y keep the token index fastest (ggml column-major [dim, T]).
//
// * T == 1 (decode): linear_gemv_kernel reads W once from HBM with 16-byte
//   loads, eight in flight per lane; the bound is HBM bandwidth over
//   M*K*4 bytes.  One wave per row (four per row when M is small, so the
//   grid still covers the chip), one cross-lane reduction per row.
// * T > 1 (prefill): linear_mfma_kernel on fp32 MFMA
//   (v_mfma_f32_32x32x2_f32); the bound is the fp32 matrix peak over
//   2*M*K*T FLOPs.  Workgroup tiles of 64x64 or 128x128 outputs, K staged
//   through LDS 32 at a time, double-buffered, one barrier per chunk.
//
// Accumulation is fp32 as in the reference; only the summation order
// differs (the reference's decode kernel reduces 256 strided partial sums,
// its prefill kernel sums k = 0..K-1 in order).
#include "common.h"
#include "launch.h"

namespace hl {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------------------
// GEMV (T == 1)
// ---------------------------------------------------------------------------
// WPR waves share one row (each takes every WPR-th 16-byte chunk); the
// workgroup's 4 waves cover 4 / WPR rows.  VEC: K % 4 == 0 and 16-byte
// aligned w and x; otherwise one float per lane per step.
template <int WPR, bool VEC>
__global__ __launch_bounds__(256) void linear_gemv_kernel(const float* __restrict__ w,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int K) {
  constexpr int RPW = 4 / WPR;
  constexpr int U = 8;  // 16-byte loads in flight per lane
  __shared__ float part[4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = blockIdx.x * RPW + wave / WPR;
  const int share = wave % WPR;
  float acc = 0.f;
  if (row < M) {
    const float* wr = w + (size_t)row * K;
    if (VEC) {
      const f32x4* w4 = (const f32x4*)wr;
      const f32x4* x4 = (const f32x4*)x;
      const int K4 = K >> 2;
      constexpr int STEP = 64 * WPR;
      float s[4] = {0.f, 0.f, 0.f, 0.f};
      int k = lane + 64 * share;
      for (; k + (U - 1) * STEP < K4; k += U * STEP) {
        f32x4 wv[U], xv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u] = w4[k + u * STEP];
#pragma unroll
        for (int u = 0; u < U; ++u) xv[u] = x4[k + u * STEP];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          s[u & 3] += wv[u].x * xv[u].x;
          s[u & 3] += wv[u].y * xv[u].y;
          s[u & 3] += wv[u].z * xv[u].z;
          s[u & 3] += wv[u].w * xv[u].w;
        }
      }
      for (; k < K4; k += STEP) {
        const f32x4 wv = w4[k], xv = x4[k];
        s[0] += wv.x * xv.x;
        s[1] += wv.y * xv.y;
        s[2] += wv.z * xv.z;
        s[3] += wv.w * xv.w;
      }
      acc = (s[0] + s[1]) + (s[2] + s[3]);
    } else {
      for (int k = lane + 64 * share; k < K; k += 64 * WPR) acc += wr[k] * x[k];
    }
  }
  acc = wave_sum(acc);
  if (WPR == 1) {
    if (lane == 0 && row < M) y[row] = acc;
  } else {
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (share == 0 && lane == 0 && row < M) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) t += part[wave + i];
      y[row] = t;
    }
  }
}

// ---------------------------------------------------------------------------
// GEMM (T > 1) on fp32 MFMA
// ---------------------------------------------------------------------------
// v_mfma_f32_32x32x2_f32: lane l supplies A[m = l%32][k = l/32] and
// B[k = l/32][n = l%32]; output element e of lane l is C[8(e/4) + 4(l/32) +
// e%4][l%32].  Within each group of 8 k, MFMA step i pairs k = 8g + i (lane
// half 0) with k = 8g + 4 + i (half 1), so a lane's four A values for the
// group are one contiguous 16-byte LDS read.
//
// The 2x2 waves of a workgroup each own a (32*WM) x (32*WN) block of the
// (64*WM) x (64*WN) output tile.
template <int WM, int WN, bool VEC>
__global__ __launch_bounds__(256) void linear_mfma_kernel(const float* __restrict__ w,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int K,
                                                          int T) {
  constexpr int BM = 64 * WM, BN = 64 * WN, BK = 32;
  // Row pitches in floats.  SA = 36: the 16 lanes served together by one
  // ds_read_b128 (rows m..m+15, same k) start on distinct 4-bank groups.
  // SB = BN + 8: rows k and k + 4 (the two lane halves of a b32 read) sit
  // 32 banks apart, so the 64 lanes hit 64 distinct banks.
  constexpr int SA = BK + 4, SB = BN + 8;
  constexpr int NA = BM * BK / 4 / 256;  // 16-byte A chunks per thread
  constexpr int NB = BK * BN / 4 / 256;  // 16-byte B chunks per thread
  __shared__ __attribute__((aligned(16))) float sA[2][BM * SA];
  __shared__ __attribute__((aligned(16))) float sB[2][BK * SB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int ln = lane & 31, hh = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  f32x4 ra[NA], rb[NB];
  auto load = [&](int c) {
    const int k0 = c * BK;
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int idx = tid + 256 * j, r = idx >> 3, kk = k0 + 4 * (idx & 7);
      const int m = m0 + r;
      if (VEC) {
        ra[j] = (m < M && kk < K) ? *(const f32x4*)(w + (size_t)m * K + kk) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ra[j][e] = (m < M && kk + e < K) ? w[(size_t)m * K + kk + e] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int idx = tid + 256 * j, r = idx / (BN / 4), n = n0 + 4 * (idx % (BN / 4));
      const int k = k0 + r;
      if (VEC) {
        rb[j] = (k < K && n < T) ? *(const f32x4*)(x + (size_t)k * T + n) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rb[j][e] = (k < K && n + e < T) ? x[(size_t)k * T + n + e] : 0.f;
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int idx = tid + 256 * j;
      *(f32x4*)&sA[buf][(idx >> 3) * SA + 4 * (idx & 7)] = ra[j];
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int idx = tid + 256 * j;
      *(f32x4*)&sB[buf][(idx / (BN / 4)) * SB + 4 * (idx % (BN / 4))] = rb[j];
    }
  };

  f32x16 acc[WM][WN];
#pragma unroll
  for (int a = 0; a < WM; ++a)
#pragma unroll
    for (int b = 0; b < WN; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  const int nk = (K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  for (int c = 0; c < nk; ++c) {
    const int buf = c & 1;
    if (c + 1 < nk) load(c + 1);
    const float* pa = &sA[buf][(wm * 32 * WM + ln) * SA + 4 * hh];
    const float* pb = &sB[buf][(4 * hh) * SB + wn * 32 * WN + ln];
#pragma unroll
    for (int g = 0; g < BK / 8; ++g) {
      f32x4 af[WM];
      float bf[WN][4];
#pragma unroll
      for (int a = 0; a < WM; ++a) af[a] = *(const f32x4*)(pa + a * 32 * SA + 8 * g);
#pragma unroll
      for (int b = 0; b < WN; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) bf[b][i] = pb[(8 * g + i) * SB + b * 32];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int a = 0; a < WM; ++a)
#pragma unroll
          for (int b = 0; b < WN; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][i], bf[b][i], acc[a][b], 0, 0, 0);
    }
    if (c + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int a = 0; a < WM; ++a)
#pragma unroll
    for (int b = 0; b < WN; ++b) {
      const int n = n0 + wn * 32 * WN + b * 32 + ln;
      if (n >= T) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 32 * WM + a * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
        if (m < M) y[(size_t)m * T + n] = acc[a][b][e];
      }
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

LinearPlan linear_plan(int M, int K, int T, const float* w, const float* x) {
  LinearPlan p{};
  if (T == 1) {
    p.gemv = true;
    p.vec = (K % 4 == 0) && aligned16(w) && aligned16(x);
    p.wpr = M >= 2048 ? 1 : 4;
    p.grid_x = (M + 4 / p.wpr - 1) / (4 / p.wpr);
    p.grid_y = 1;
  } else {
    p.gemv = false;
    p.vec = (K % 4 == 0) && (T % 4 == 0) && aligned16(w) && aligned16(x);
    const long long big = (long long)((M + 127) / 128) * ((T + 127) / 128);
    p.tile = big >= 512 ? 128 : 64;
    p.grid_x = (T + p.tile - 1) / p.tile;
    p.grid_y = (M + p.tile - 1) / p.tile;
  }
  return p;
}

hipError_t linear_col_launch(float* y, const float* x, const float* w, int K, int M, int T,
                             hipStream_t stream) {
  const LinearPlan p = linear_plan(M, K, T, w, x);
  const dim3 grid(p.grid_x, p.grid_y), block(256);
  if (p.gemv) {
    if (p.wpr == 1) {
      if (p.vec) hipLaunchKernelGGL((linear_gemv_kernel<1, true>), grid, block, 0, stream, w, x, y, M, K);
      else hipLaunchKernelGGL((linear_gemv_kernel<1, false>), grid, block, 0, stream, w, x, y, M, K);
    } else {
      if (p.vec) hipLaunchKernelGGL((linear_gemv_kernel<4, true>), grid, block, 0, stream, w, x, y, M, K);
      else hipLaunchKernelGGL((linear_gemv_kernel<4, false>), grid, block, 0, stream, w, x, y, M, K);
    }
  } else if (p.tile == 128) {
    if (p.vec) hipLaunchKernelGGL((linear_mfma_kernel<2, 2, true>), grid, block, 0, stream, w, x, y, M, K, T);
    else hipLaunchKernelGGL((linear_mfma_kernel<2, 2, false>), grid, block, 0, stream, w, x, y, M, K, T);
  } else {
    if (p.vec) hipLaunchKernelGGL((linear_mfma_kernel<1, 1, true>), grid, block, 0, stream, w, x, y, M, K, T);
    else hipLaunchKernelGGL((linear_mfma_kernel<1, 1, false>), grid, block, 0, stream, w, x, y, M, K, T);
  }
  return hipGetLastError();
}

}  // namespace hl
