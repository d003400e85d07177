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
// Smallest magnitude that rounds (RNE) to an fp16 infinity.
constexpr float kF16Inf = 65520.0f;

// Range record of an fp16-operand prefill: four words in the workspace,
// written and read only by the kernels of the prefill's launch sequence.
// Each word is written in a kernel where no other workgroup reads it, so
// stream order alone orders every access (plain loads and stores: a later
// kernel sees an earlier kernel's stores).
//   [0] F  overflow mark: G + 1 when this call met an operand >= 65520
//   [1] G  call generation, advanced by the last kernel of each call
//   [2] S  G + 1, staged by the fallback prologue for the fallback kernel
//   [3] O  1 when the last call took the fallback, else 0
// A stale F (from an earlier call) differs from G + 1 because G has moved
// on since; a zero-filled record reads as "no overflow".
// An operand of this call overflowed fp16 (prologue and flash kernel).
__device__ __forceinline__ void range_flag_set(unsigned* rec) { rec[0] = rec[1] + 1u; }

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32 under the default RNE mode
  return __builtin_bit_cast(uint16_t, h);
}

// fp8 e4m3 (OCP "e4m3fn"): round to nearest even, saturating to +-448
// (infinities included), NaN -> NaN; identical on host and device.
__host__ __device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);   // NaN
  if (a >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);  // >= 448 (and inf): saturate
  if (a >= 0x3C800000u) {                                // >= 2^-6: normal
    const uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);  // round off 20 mantissa bits
    uint32_t v = (r >> 20) - (120u << 3);                // rebias 127 -> 7
    if (v > 0x7Eu) v = 0x7Eu;
    return (uint8_t)(sign | v);
  }
  // subnormal: m * 2^-9, m = round-to-even(|f| * 512) in 0..8 (8 = 2^-6)
  float af;
  __builtin_memcpy(&af, &a, 4);
  const float s = af * 512.0f;  // exact: power-of-two scaling of a value < 8
  uint32_t m = (uint32_t)s;
  const float fr = s - (float)m;
  if (fr > 0.5f || (fr == 0.5f && (m & 1u))) ++m;
  return (uint8_t)(sign | m);
}
// Exact decode through the hardware conversion (v_cvt_scalef32_pk_f16_fp8
// with scale 1 reproduces every e4m3fn code, NaN included).
__device__ __forceinline__ uint16_t e4m3_to_f16_bits(uint8_t b) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((uint32_t)b, 1.0f, false);
  return __builtin_bit_cast(uint16_t, (_Float16)v[0]);
}
// Eight e4m3 values (bytes of lo, then hi) to eight fp16 bit patterns.
__device__ __forceinline__ u16x8 e4m3x8_to_f16x8(uint32_t lo, uint32_t hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
  const h2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
  const h2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
  const h2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v w = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                    __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
  return __builtin_bit_cast(u16x8, w);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == HL_F32) return ((const float*)p)[i];
  else if constexpr (DT == HL_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == HL_FP8) return f16_bits_to_f32(e4m3_to_f16_bits(((const uint8_t*)p)[i]));
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
  else if constexpr (DT == HL_FP8) ((uint8_t*)p)[i] = f32_to_e4m3(v);
  else ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}
// 16-bit working form of a stored value: the storage bits for fp16/bf16; for
// fp8 the fp16 bits of the e4m3-rounded value (exact), which is how fp8
// caches enter the fp16 MFMAs.
template <int DT>
__device__ __forceinline__ uint16_t to_bits(float v) {
  if constexpr (DT == HL_F16) return f32_to_f16_bits(v);
  else if constexpr (DT == HL_FP8) return e4m3_to_f16_bits(f32_to_e4m3(v));
  else return f32_to_bf16_bits(v);
}
template <int DT>
__device__ __forceinline__ float from_bits(uint16_t b) {
  if constexpr (DT == HL_F16 || DT == HL_FP8) return f16_bits_to_f32(b);
  else return bf16_bits_to_f32(b);
}
// Bytes per stored element.
template <int DT>
constexpr int elem_bytes() { return DT == HL_F32 ? 4 : (DT == HL_FP8 ? 1 : 2); }

// Offset of element (row d, column t) inside one kv head's cache block
// (the block starts at h * D * max_len in either layout): column-major rows
// of max_len, or max_len/32 tiles of [D][32].
__host__ __device__ __forceinline__ int64_t kv_off(int layout, int d, int t, int D, int max_len) {
  return layout == HL_KV_TILED32 ? ((int64_t)(t >> 5) * D + d) * 32 + (t & 31)
                                 : (int64_t)d * max_len + t;
}

// Paged caches (HL_KV_PAGED32): offset of element (d, t) of kv head h of
// sequence b in the pool, through that sequence's row of the block table.
__device__ __forceinline__ int64_t kv_paged_off(const int* table, int bps, int b, int n_head_kv, int h,
                                                int D, int d, int t) {
  const int64_t page = table[(int64_t)b * bps + (t >> 5)];
  return page * ((int64_t)n_head_kv * D * 32) + ((int64_t)h * D + d) * 32 + (t & 31);
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

// cos and sin of a RoPE angle (up to ~max_len rad): one sincosf shares the
// large-argument range reduction that separate cosf / sinf calls each repeat.
__device__ __forceinline__ void rope_cs(float angle, float& c, float& s) { sincosf(angle, &s, &c); }

// RoPE angle table passed by value as a kernel argument (no device memory).
struct ThetaTable {
  float t[HL_MAX_ROPE_DIM / 2];
};

// Split of fp32 operands into fp16 hi + lo * 2^-11 for three-MFMA
// products (the fp32 prefill).
// x ~= hi + lo * 2^-11 with hi, lo fp16: |x - hi - lo 2^-11| <= |x| 2^-22
// for |x| < 32768 with hi normal (2^-36 absolute below fp16's normal range).
// hi * hi' + (hi * lo' + lo * hi') 2^-11 is then the product to ~2^-21.
__device__ __forceinline__ void split_f16x8(const float* x, f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const _Float16 h = (_Float16)x[j];
    hi[j] = h;
    lo[j] = (_Float16)((x[j] - (float)h) * 2048.f);
  }
}
// Power-of-two exponent that brings a magnitude (given as its bit pattern,
// finite) into [2^13, 2^14): split operands scaled by it keep their hi parts
// in fp16's normal range (the matrix cores treat fp16 subnormals as zero)
// for every element within 2^27 of the largest.  0 for an all-zero set.
__device__ __forceinline__ int split_shift(uint32_t max_bits) {
  if (max_bits == 0u) return 0;
  const int e = max_bits >= 0x00800000u ? (int)(max_bits >> 23) - 127 : -127;
  return 13 - e;
}
constexpr uint32_t kInfBits = 0x7F800000u;  // |x| bit patterns at or above: inf or NaN
// Split images of the fp32 prefill (head dim D = 64 or 128), one per (kv
// head, 64-key tile): K hi, K lo ([key][D] fp16, 16-byte chunk c of key j at
// c ^ (j % (D / 8))), V hi, V lo ([d][64 keys] fp16, chunk c of dim d at
// c ^ ((d / 2) % 8)).  Each 32-key half of a tile has its own power-of-two
// scale per tensor; the tile's record holds 8 ints: the K shifts of halves
// 0 and 1, the V shifts, then inf/NaN flags of K halves 0, 1 and V halves.
constexpr int split_img_bytes(int D) { return 64 * D * 8; }
constexpr int kSplitRecInts = 8;

}  // namespace hl
