// Quantized decode GEMV over GGUF weight rows: the drop-in for
// gpuLinearColQuant (backends/naive.nim:1580-1592) for the formats most GGUF
// models use: F16, Q8_0, Q4_K and Q6_K (dequantisation as in the reference's
// quant.nim: dequantRowQ8_0 :304-319, dequantRowQ4K :235-277,
// dequantRowQ6K :321-355, halfToFloat :78-96).
//
//   y[M] = dequant(W)[M, K] . x[K]      (seq_len 1, like the reference)
//
// HBM-bound on the quantized bytes (Q4_K: 144 B per 256 weights).  One wave
// per row (four per row when M is small); a row streams through LDS in
// chunks of whole blocks: every lane loads dwords of the chunk (coalesced,
// whatever the block size: Q8_0 blocks are 34 bytes, Q6_K 210), the next
// chunk's dwords are in flight while the current one is decoded.  Lanes
// decode 32-element sub-blocks (16 elements for F16) and dot them with x;
// per-block scale and min factor out of the inner sums.  Rows whose byte
// size is not a multiple of 4 (Q8_0 with K % 64, Q6_K with K % 512) load
// bytes instead of dwords.
#include "common.h"
#include "launch.h"

namespace hl {
namespace {

template <int QT>
struct QFmt;
template <>
struct QFmt<1> {  // F16
  static constexpr int QK = 32, BYTES = 64, SUB = 2, CHUNK = 32;  // "block" = 32 halfs
};
template <>
struct QFmt<8> {  // Q8_0: fp16 d, 32 x int8
  static constexpr int QK = 32, BYTES = 34, SUB = 1, CHUNK = 64;
};
template <>
struct QFmt<12> {  // Q4_K: fp16 d, fp16 dmin, 12 bytes 6-bit scales/mins, 128 bytes nibbles
  static constexpr int QK = 256, BYTES = 144, SUB = 8, CHUNK = 16;
};
template <>
struct QFmt<14> {  // Q6_K: 128 bytes ql, 64 bytes qh, 16 int8 scales, fp16 d
  static constexpr int QK = 256, BYTES = 210, SUB = 8, CHUNK = 12;
};

__device__ __forceinline__ float half_at(const uint8_t* p) {
  return f16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

// Sum over 32 consecutive x values starting at xs (16-byte aligned when V4).
template <bool V4>
__device__ __forceinline__ void load_x32(const float* xs, float* xv) {
  if (V4) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 v = *(const f32x4*)(xs + 4 * i);
      xv[4 * i] = v.x;
      xv[4 * i + 1] = v.y;
      xv[4 * i + 2] = v.z;
      xv[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) xv[i] = xs[i];
  }
}

// Contribution of sub-block `sub` of block `blk` (its bytes at bp) to the dot
// product with x (the block's first element at xb).
template <int QT, bool V4>
__device__ __forceinline__ float sub_dot(const uint8_t* bp, int sub, const float* xb) {
  if constexpr (QT == 1) {  // F16: sub s covers halfs 16s .. 16s+15
    float acc = 0.f;
    const float* xs = xb + 16 * sub;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += half_at(bp + 2 * (16 * sub + i)) * xs[i];
    return acc;
  } else if constexpr (QT == 8) {  // Q8_0: d * sum(q * x)
    float xv[32];
    load_x32<V4>(xb, xv);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s += (float)(int8_t)bp[2 + i] * xv[i];
    return half_at(bp) * s;
  } else if constexpr (QT == 12) {
    // Q4_K sub j: elements 32j .. 32j+31, nibbles of bytes 16 + 32(j/2) + l
    // (low for even j, high for odd), scale/min pair j (getScaleMinK4).
    const float d = half_at(bp), dmin = half_at(bp + 2);
    const uint8_t* sc = bp + 4;
    int scv, mnv;
    if (sub < 4) {
      scv = sc[sub] & 63;
      mnv = sc[sub + 4] & 63;
    } else {
      scv = (sc[sub + 4] & 0x0F) | ((sc[sub - 4] >> 6) << 4);
      mnv = (sc[sub + 4] >> 4) | ((sc[sub] >> 6) << 4);
    }
    const uint8_t* q = bp + 16 + 32 * (sub >> 1);
    const int sh = 4 * (sub & 1);
    float xv[32];
    load_x32<V4>(xb + 32 * sub, xv);
    float sq = 0.f, sx = 0.f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      sq += (float)((q[l] >> sh) & 0x0F) * xv[l];
      sx += xv[l];
    }
    return d * (float)scv * sq - dmin * (float)mnv * sx;
  } else {
    // Q6_K sub j = 4n + t: elements 128n + 32t + l; low 4 bits from
    // ql[64n + 32(t&1) + l] (nibble t>>1), high 2 bits from qh[32n + l]
    // (bits 2t), scale sc[8n + 2t + l/16], minus 32.
    const int n = sub >> 2, t = sub & 3;
    const uint8_t* ql = bp + 64 * n + 32 * (t & 1);
    const uint8_t* qh = bp + 128 + 32 * n;
    const int8_t* sc = (const int8_t*)(bp + 192) + 8 * n + 2 * t;
    const float d = half_at(bp + 208);
    const int shl = 4 * (t >> 1), shh = 2 * t;
    float xv[32];
    load_x32<V4>(xb + 128 * n + 32 * t, xv);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const int q = (((ql[l] >> shl) & 0x0F) | (((qh[l] >> shh) & 3) << 4)) - 32;
      if (l < 16) s0 += (float)q * xv[l];
      else s1 += (float)q * xv[l];
    }
    return d * ((float)sc[0] * s0 + (float)sc[1] * s1);
  }
}

// WPR waves per row (1 or 4).  ALIGNED: row byte size % 4 == 0 and w 4-byte
// aligned (dword loads); V4: x 16-byte aligned.
template <int QT, int WPR, bool ALIGNED, bool V4>
__global__ __launch_bounds__(256) void quant_gemv_kernel(const uint8_t* __restrict__ w,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int M, int K) {
  using F = QFmt<QT>;
  constexpr int NB = F::CHUNK;                    // blocks per chunk
  constexpr int CB = NB * F::BYTES;               // chunk bytes
  constexpr int CDW = (CB + 3) / 4;               // chunk dwords
  constexpr int PL = (CDW + 63) / 64;             // dwords per lane per chunk
  constexpr int RPW = 4 / WPR;                    // rows per workgroup
  __shared__ __attribute__((aligned(16))) uint32_t sbuf[4][PL * 64];
  __shared__ float part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * RPW + wave / WPR;
  const int share = wave % WPR;
  const int nb = K / F::QK;
  const long long rowbytes = (long long)nb * F::BYTES;
  const int nchunks = (nb + NB - 1) / NB;
  float acc = 0.f;
  if (row < M) {
    const uint8_t* wr = w + (long long)row * rowbytes;
    uint8_t* lds = (uint8_t*)sbuf[wave];
    uint32_t regs[PL];
    // chunk c (of this wave's share) -> registers
    auto load = [&](int c) {
      const long long cb0 = (long long)c * CB;
      const int valid = (int)min((long long)CB, rowbytes - cb0);
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        const int dw = lane + 64 * i;
        if (ALIGNED) {
          regs[i] = 4 * dw < valid ? *(const uint32_t*)(wr + cb0 + 4 * dw) : 0u;
        } else {
          uint32_t v = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (4 * dw + e < valid) v |= (uint32_t)wr[cb0 + 4 * dw + e] << (8 * e);
          regs[i] = v;
        }
      }
    };
    int c = share;
    if (c < nchunks) load(c);
    for (; c < nchunks; c += WPR) {
#pragma unroll
      for (int i = 0; i < PL; ++i) sbuf[wave][lane + 64 * i] = regs[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (c + WPR < nchunks) load(c + WPR);  // next chunk in flight while this one is decoded
      const int b0 = c * NB;
      const int nbc = min(NB, nb - b0);
      for (int u = lane; u < nbc * F::SUB; u += 64) {
        const int blk = u / F::SUB, sub = u % F::SUB;
        acc += sub_dot<QT, V4>(lds + blk * F::BYTES, sub, x + (long long)(b0 + blk) * F::QK);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
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

template <int QT, int WPR>
void launch_q(const uint8_t* w, const float* x, float* y, int M, int K, bool aligned, bool v4,
              hipStream_t stream) {
  const dim3 grid((M + 4 / WPR - 1) / (4 / WPR)), block(256);
  if (aligned) {
    if (v4) hipLaunchKernelGGL((quant_gemv_kernel<QT, WPR, true, true>), grid, block, 0, stream, w, x, y, M, K);
    else hipLaunchKernelGGL((quant_gemv_kernel<QT, WPR, true, false>), grid, block, 0, stream, w, x, y, M, K);
  } else {
    if (v4) hipLaunchKernelGGL((quant_gemv_kernel<QT, WPR, false, true>), grid, block, 0, stream, w, x, y, M, K);
    else hipLaunchKernelGGL((quant_gemv_kernel<QT, WPR, false, false>), grid, block, 0, stream, w, x, y, M, K);
  }
}

template <int QT>
void launch_qt(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t stream) {
  const long long rowbytes = (long long)(K / QFmt<QT>::QK) * QFmt<QT>::BYTES;
  const bool aligned = rowbytes % 4 == 0 && ((uintptr_t)w & 3) == 0;
  const bool v4 = ((uintptr_t)x & 15) == 0;
  if (M >= 2048) launch_q<QT, 1>(w, x, y, M, K, aligned, v4, stream);
  else launch_q<QT, 4>(w, x, y, M, K, aligned, v4, stream);
}

}  // namespace

int quant_block_elems(int qtype) {
  switch (qtype) {
    case HL_GGML_F16: return 32;
    case HL_GGML_Q8_0: return 32;
    case HL_GGML_Q4_K: return 256;
    case HL_GGML_Q6_K: return 256;
    default: return 0;
  }
}

long long quant_row_bytes(int qtype, int K) {
  switch (qtype) {
    case HL_GGML_F16: return 2LL * K;
    case HL_GGML_Q8_0: return (long long)(K / 32) * 34;
    case HL_GGML_Q4_K: return (long long)(K / 256) * 144;
    case HL_GGML_Q6_K: return (long long)(K / 256) * 210;
    default: return 0;
  }
}

hipError_t linear_quant_launch(float* y, const float* x, const void* w, int K, int M, int qtype,
                               hipStream_t stream) {
  const uint8_t* wb = (const uint8_t*)w;
  switch (qtype) {
    case HL_GGML_F16: launch_qt<1>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q8_0: launch_qt<8>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q4_K: launch_qt<12>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q6_K: launch_qt<14>(wb, x, y, M, K, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace hl
