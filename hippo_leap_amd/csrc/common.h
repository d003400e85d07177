// Shared device/host helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hl_attn.h"

namespace hl {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Storage conversions.  Upcasts are exact; downcasts round to nearest even.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;  // v_cvt_f32_f16: exact, keeps inf/nan/subnormals
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32 under the default RNE mode
  return __builtin_bit_cast(uint16_t, h);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == HL_F32) return ((const float*)p)[i];
  else if constexpr (DT == HL_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  else return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  // Materialise the fp32 value first: without the barrier the compiler may
  // fuse the producing multiply into a mixed-precision op that rounds once
  // to 16 bits, which is not the RNE of the fp32 result.
  if constexpr (DT != HL_F32) __asm__ volatile("" : "+v"(v));
  if constexpr (DT == HL_F32) ((float*)p)[i] = v;
  else if constexpr (DT == HL_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}
template <int DT>
__device__ __forceinline__ uint16_t to_bits(float v) {
  if constexpr (DT == HL_F16) return f32_to_f16_bits(v);
  else return f32_to_bf16_bits(v);
}
template <int DT>
__device__ __forceinline__ float from_bits(uint16_t b) {
  if constexpr (DT == HL_F16) return f16_bits_to_f32(b);
  else return bf16_bits_to_f32(b);
}

// Offset of element (row d, column t) inside one kv head's cache block
// (the block starts at h * D * max_len in either layout): column-major rows
// of max_len, or max_len/32 tiles of [D][32].
__host__ __device__ __forceinline__ int64_t kv_off(int layout, int d, int t, int D, int max_len) {
  return layout == HL_KV_TILED32 ? ((int64_t)(t >> 5) * D + d) * 32 + (t & 31)
                                 : (int64_t)d * max_len + t;
}

// ---------------------------------------------------------------------------
// Wave64 reductions (xor butterflies over ds_swizzle / DPP via __shfl_xor).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// RoPE angle table passed by value as a kernel argument (no device memory).
struct ThetaTable {
  float t[HL_MAX_ROPE_DIM / 2];
};

}  // namespace hl
