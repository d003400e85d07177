// One head vector of the new decode token, processed by one wave in LDS:
// optional RMSNorm, then optional RoPE at `pos`.  Shared by the stand-alone
// qkNorm/RoPE/store kernel and the fused decode-step attention kernel, so
// both produce the same bits.
//
// Formulas kept from the reference:
//   RMSNorm   x * (1/sqrtf(sum(x^2)/D + eps)) * w[d]          (naive.nim:2910, :2915)
//   RoPE      angle = float(pos) * theta[i];                    (naive.nim:3065-3073)
//             (v0, v1) -> (v0*c - v1*s, v0*s + v1*c)
//             half-split pairs (i, i+rope_dim/2), or interleaved (2i, 2i+1)
//             as in tensor.nim:156-166; dims >= rope_dim pass through
#pragma once

#include "common.h"

namespace hl {

__device__ __forceinline__ void rope_pair_index(int i, int half, int style, int& i0, int& i1) {
  if (style == HL_ROPE_HALF_SPLIT) {
    i0 = i;
    i1 = i + half;
  } else {
    i0 = 2 * i;
    i1 = 2 * i + 1;
  }
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The two halves of the per-head work, shared so that every kernel that
// applies them produces the same bits.  No FMA contraction: each product and
// sum is rounded on its own, whatever the calling kernel's schedule.

// Sum of squares -> 1/sqrtf(mean + eps); `ss` is this lane's partial sum
// over its elements in ascending d.
__device__ __forceinline__ float rms_inv(float ss, int D, float eps) {
#pragma clang fp contract(off)
  ss = wave_sum(ss);
  return 1.0f / sqrtf(ss / (float)D + eps);
}
__device__ __forceinline__ float sq_acc(float ss, float x) {
#pragma clang fp contract(off)
  return ss + x * x;
}
__device__ __forceinline__ float norm_apply(float x, float inv, float w) {
#pragma clang fp contract(off)
  return x * inv * w;
}
// Rotation of pair i of an LDS head vector by (c, s) = (cos, sin) of its angle.
__device__ __forceinline__ void rope_rotate(float* sx, int i, int half, int style, float c, float s) {
#pragma clang fp contract(off)
  int i0, i1;
  rope_pair_index(i, half, style, i0, i1);
  const float v0 = sx[i0], v1 = sx[i1];
  sx[i0] = v0 * c - v1 * s;
  sx[i1] = v0 * s + v1 * c;
}

// sx: D floats in LDS, already loaded and visible to the wave.  nw == null:
// no norm; rope_dim == 0: no RoPE.
__device__ __forceinline__ void headvec_norm_rope(float* sx, int D, int lane, const float* nw, float eps,
                                                  int rope_dim, int rope_style, const ThetaTable& theta,
                                                  int pos) {
  if (nw) {
    float ss = 0.f;
    for (int d = lane; d < D; d += 64) ss = sq_acc(ss, sx[d]);
    const float inv = rms_inv(ss, D, eps);
    for (int d = lane; d < D; d += 64) sx[d] = norm_apply(sx[d], inv, nw[d]);
    wave_lds_sync();
  }
  if (rope_dim > 0) {
    const int half = rope_dim / 2;
    for (int i = lane; i < half; i += 64) {
      const float angle = (float)pos * theta.t[i];
      float c, sn;
      rope_cs(angle, c, sn);
      rope_rotate(sx, i, half, rope_style, c, sn);
    }
    wave_lds_sync();
  }
}

}  // namespace hl
