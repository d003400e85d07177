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
// * T == 1 (decode): linear_gemv_kernel reads W once from HBM with
//   non-temporal 16-byte loads, eight in flight per lane; the bound is HBM
//   bandwidth over M*K*4 bytes.  One wave per row (four per row when M is
//   small, so the grid still covers the chip), one cross-lane reduction per
//   row.  x is re-read from L2 by every wave (staging it in LDS measured
//   slower).
// * T > 1 (prefill): linear_mfma_kernel on fp32 MFMA
//   (v_mfma_f32_32x32x2_f32); the bound is the fp32 matrix peak over
//   2*M*K*T FLOPs.  Workgroup tiles of 128x128 outputs (4 waves, 2x2 blocks
//   of 32x32 each) when there are enough of them to fill the chip, else
//   64x64 (8 waves in two K halves); K staged through double-buffered LDS
//   with two chunks in flight in registers, one barrier per chunk.
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
        for (int u = 0; u < U; ++u)
          wv[u] = __builtin_nontemporal_load(&w4[k + u * STEP]);  // W is read once
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
        const f32x4 wv = __builtin_nontemporal_load(&w4[k]), xv = x4[k];
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
// (64*WM) x (64*WN) output tile.  KW = 2 doubles the workgroup to 8 waves:
// waves 4..7 take the upper half of every K chunk for the same blocks (two
// waves per SIMD to cover each other's LDS and barrier waits), and their
// sums are added through LDS at the end.
template <int WM, int WN, int BK, int KW, bool VEC, int PF = 2>
__global__ __launch_bounds__(256 * KW) void linear_mfma_kernel(const float* __restrict__ w,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ y, int M, int K,
                                                          int T) {
  constexpr int BM = 64 * WM, BN = 64 * WN;
  // Row pitches in floats.  SA = 36: the 16 lanes served together by one
  // ds_read_b128 (rows m..m+15, same k) start on distinct 4-bank groups.
  // SB = BN + 8: rows k and k + 4 (the two lane halves of a b32 read) sit
  // 32 banks apart, so the 64 lanes hit 64 distinct banks.
  constexpr int SA = BK + 4, SB = BN + 8;
  constexpr int NTH = 256 * KW;
  constexpr int NA = BM * BK / 4 / NTH;  // 16-byte A chunks per thread
  constexpr int NB = BK * BN / 4 / NTH;  // 16-byte B chunks per thread
  static_assert(NA * NTH * 4 == BM * BK && NB * NTH * 4 == BK * BN, "tile / thread mismatch");
  __shared__ __attribute__((aligned(16))) float sA[2][BM * SA];
  __shared__ __attribute__((aligned(16))) float sB[2][BK * SB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int ln = lane & 31, hh = lane >> 5;
  const int kg = wave >> 2;  // K half of each chunk (KW = 2)
  const int wm = (wave >> 1) & 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  f32x4 ra[PF][NA], rb[PF][NB];  // PF chunks in flight, one register set each
  auto load = [&](int c, int st) {
    const int k0 = c * BK;
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int idx = tid + NTH * j, r = idx / (BK / 4), kk = k0 + 4 * (idx % (BK / 4));
      const int m = m0 + r;
      if (VEC) {
        ra[st][j] = (m < M && kk < K) ? *(const f32x4*)(w + (size_t)m * K + kk) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ra[st][j][e] = (m < M && kk + e < K) ? w[(size_t)m * K + kk + e] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int idx = tid + NTH * j, r = idx / (BN / 4), n = n0 + 4 * (idx % (BN / 4));
      const int k = k0 + r;
      if (VEC) {
        rb[st][j] = (k < K && n < T) ? *(const f32x4*)(x + (size_t)k * T + n) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rb[st][j][e] = (k < K && n + e < T) ? x[(size_t)k * T + n + e] : 0.f;
      }
    }
  };
  auto store = [&](int buf, int st) {
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int idx = tid + NTH * j;
      *(f32x4*)&sA[buf][(idx / (BK / 4)) * SA + 4 * (idx % (BK / 4))] = ra[st][j];
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int idx = tid + NTH * j;
      *(f32x4*)&sB[buf][(idx / (BN / 4)) * SB + 4 * (idx % (BN / 4))] = rb[st][j];
    }
  };

  // Independent accumulation chains per output block: back-to-back MFMAs
  // into one accumulator wait for each other, so with a single 32x32 block
  // per wave the k-steps rotate over CH accumulators (summed at the end).
  constexpr int CH = (WM * WN >= 2) ? 1 : 2;
  f32x16 acc[WM][WN][CH];
#pragma unroll
  for (int a = 0; a < WM; ++a)
#pragma unroll
    for (int b = 0; b < WN; ++b)
#pragma unroll
      for (int h = 0; h < CH; ++h)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][h][e] = 0.f;

  auto compute = [&](int buf) {
    const float* pa = &sA[buf][(wm * 32 * WM + ln) * SA + 4 * hh];
    const float* pb = &sB[buf][(4 * hh) * SB + wn * 32 * WN + ln];
    constexpr int GPW = BK / 8 / KW;  // groups of 8 k per wave and chunk
#pragma unroll
    for (int g = kg * GPW; g < (kg + 1) * GPW; ++g) {
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
            acc[a][b][i % CH] =
                __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][i], bf[b][i], acc[a][b][i % CH], 0, 0, 0);
    }
  };

  // Chunk j travels in register set j % PF: chunks 0..PF-1 are requested up
  // front, and each iteration refills the set it has just written to LDS
  // with the chunk PF further on.
  const int nk = (K + BK - 1) / BK;
#pragma unroll
  for (int st = 0; st < PF; ++st)
    if (st < nk) load(st, st);
  store(0, 0);
  if (PF < nk) load(PF, 0);
  __syncthreads();
  for (int c0 = 0; c0 < nk; c0 += PF) {
#pragma unroll
    for (int q = 0; q < PF; ++q) {
      const int c = c0 + q;
      if (c < nk) {
        compute(c & 1);
        const int st = (q + 1) % PF;
        if (c + 1 < nk) store((c + 1) & 1, st);
        if (c + 1 + PF < nk) load(c + 1 + PF, st);
        __syncthreads();
      }
    }
  }

  float* red = sA[0];  // KW = 2: the upper waves' sums, [wave][a][b][e][lane]
  if (KW == 2 && kg == 1) {
#pragma unroll
    for (int a = 0; a < WM; ++a)
#pragma unroll
      for (int b = 0; b < WN; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float v = acc[a][b][0][e];
#pragma unroll
          for (int h = 1; h < CH; ++h) v += acc[a][b][h][e];
          red[((((wave & 3) * WM + a) * WN + b) * 16 + e) * 64 + lane] = v;
        }
  }
  if (KW == 2) __syncthreads();
  if (kg == 1) return;
#pragma unroll
  for (int a = 0; a < WM; ++a)
#pragma unroll
    for (int b = 0; b < WN; ++b) {
      const int n = n0 + wn * 32 * WN + b * 32 + ln;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 32 * WM + a * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
        float v = acc[a][b][0][e];
#pragma unroll
        for (int h = 1; h < CH; ++h) v += acc[a][b][h][e];
        if (KW == 2) v += red[(((wave * WM + a) * WN + b) * 16 + e) * 64 + lane];
        if (m < M && n < T) y[(size_t)m * T + n] = v;
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
    if (p.vec) hipLaunchKernelGGL((linear_mfma_kernel<2, 2, 32, 1, true>), grid, block, 0, stream, w, x, y, M, K, T);
    else hipLaunchKernelGGL((linear_mfma_kernel<2, 2, 32, 1, false>), grid, block, 0, stream, w, x, y, M, K, T);
  } else {
    if (p.vec) hipLaunchKernelGGL((linear_mfma_kernel<1, 1, 64, 2, true>), grid, dim3(512), 0, stream, w, x, y, M, K, T);
    else hipLaunchKernelGGL((linear_mfma_kernel<1, 1, 64, 2, false>), grid, dim3(512), 0, stream, w, x, y, M, K, T);
  }
  return hipGetLastError();
}

}  // namespace hl
