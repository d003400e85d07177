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
#include <algorithm>

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
template <>
struct QFmt<6> {  // Q5_0: fp16 d, 32 high bits, 16 nibble bytes
  static constexpr int QK = 32, BYTES = 22, SUB = 1, CHUNK = 64;
};
template <>
struct QFmt<7> {  // Q5_1: fp16 d, fp16 m, 32 high bits, 16 nibble bytes
  static constexpr int QK = 32, BYTES = 24, SUB = 1, CHUNK = 64;
};
template <>
struct QFmt<20> {  // IQ4_NL: fp16 d, 16 nibble bytes indexing a level table
  static constexpr int QK = 32, BYTES = 18, SUB = 1, CHUNK = 64;
};
template <>
struct QFmt<10> {  // Q2_K: 16 scale/min bytes, 64 bytes of 2-bit quants, d, dmin
  static constexpr int QK = 256, BYTES = 84, SUB = 8, CHUNK = 16;
};
template <>
struct QFmt<11> {  // Q3_K: hmask[32], qs[64], 12 bytes of 6-bit scales, fp16 d
  static constexpr int QK = 256, BYTES = 110, SUB = 8, CHUNK = 16;
};
template <>
struct QFmt<13> {  // Q5_K: d, dmin, 12 scale bytes, qh[32], qs[128]
  static constexpr int QK = 256, BYTES = 176, SUB = 8, CHUNK = 16;
};

// The IQ4_NL format's 16 non-linear levels (quant.nim:16-17), as int8 bytes
// of four dwords, looked up in registers with v_perm_b32: selector byte s
// picks byte s of {hi:lo} (0-3 from lo, 4-7 from hi).
__device__ __forceinline__ float iq4nl_level(uint32_t idx) {
  constexpr uint32_t T0 = 0xBFAD9881u;  // -127, -104, -83, -65
  constexpr uint32_t T1 = 0xF6EADDCFu;  //  -49,  -35, -22, -10
  constexpr uint32_t T2 = 0x26190D01u;  //    1,   13,  25,  38
  constexpr uint32_t T3 = 0x71594535u;  //   53,   69,  89, 113
  const uint32_t lo = __builtin_amdgcn_perm(T1, T0, idx & 7u);
  const uint32_t hi = __builtin_amdgcn_perm(T3, T2, idx & 7u);
  return (float)(int8_t)(((idx & 8u) ? hi : lo) & 255u);
}

// Four IQ4_NL levels at once: n4 holds one level index (0-15) per byte.
__device__ __forceinline__ uint32_t iq4nl_levels4(uint32_t n4) {
  constexpr uint32_t T0 = 0xBFAD9881u, T1 = 0xF6EADDCFu, T2 = 0x26190D01u, T3 = 0x71594535u;
  const uint32_t sel = n4 & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
  const uint32_t m = ((n4 >> 3) & 0x01010101u) * 0xFFu;  // 0xFF in bytes with index >= 8
  return (lo & ~m) | (hi & m);
}

__device__ __forceinline__ uint32_t u32_at(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// getScaleMinK4 (quant.nim:235-242): 6-bit scale / min j of the 12 bytes.
__device__ __forceinline__ void scale_min_k4(const uint8_t* sc, int j, int& scv, int& mnv) {
  if (j < 4) {
    scv = sc[j] & 63;
    mnv = sc[j + 4] & 63;
  } else {
    scv = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
    mnv = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
  }
}

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
  } else if constexpr (QT == 6 || QT == 7 || QT == 20) {
    // One 32-element block: element j < 16 = low nibble of qs[j], element
    // 16 + j = its high nibble; Q5_0 / Q5_1 add bit j of qh as bit 4.
    constexpr int QS = QT == 6 ? 6 : QT == 7 ? 8 : 2;
    const uint32_t qh = QT == 6 ? u32_at(bp + 2) : QT == 7 ? u32_at(bp + 4) : 0u;
    float xv[32];
    load_x32<V4>(xb, xv);
    float sq = 0.f, sx = 0.f;
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      const int b = bp[QS + l];
      if constexpr (QT == 20) {
        sq += iq4nl_level((uint32_t)b & 15u) * xv[l] + iq4nl_level((uint32_t)b >> 4) * xv[16 + l];
      } else {
        const int q0 = (b & 15) | (int)(((qh >> l) & 1u) << 4);
        const int q1 = (b >> 4) | (int)(((qh >> (l + 16)) & 1u) << 4);
        sq += (float)q0 * xv[l] + (float)q1 * xv[16 + l];
        sx += xv[l] + xv[16 + l];
      }
    }
    const float d = half_at(bp);
    if constexpr (QT == 6) return d * (sq - 16.f * sx);  // d * (q - 16)
    else if constexpr (QT == 7) return d * sq + half_at(bp + 2) * sx;  // d * q + m
    else return d * sq;
  } else if constexpr (QT == 10 || QT == 11) {
    // Q2_K / Q3_K sub k = 4n + j: elements 32k + l, bits 2j of
    // qs[32n + l]; scale 8n + 2j + (l >= 16).  Q3_K subtracts 4 unless bit
    // 4n + j of hmask[l] is set, and its scales are 6-bit minus 32.
    const int n = sub >> 2, j = sub & 3;
    const uint8_t* qs = bp + (QT == 10 ? 16 : 32) + 32 * n;
    float xv[32];
    load_x32<V4>(xb + 32 * sub, xv);
    float s0 = 0.f, s1 = 0.f, x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      int q = (qs[l] >> (2 * j)) & 3;
      if constexpr (QT == 11) q -= ((bp[l] >> (4 * n + j)) & 1) ? 0 : 4;
      if (l < 16) { s0 += (float)q * xv[l]; x0 += xv[l]; }
      else { s1 += (float)q * xv[l]; x1 += xv[l]; }
    }
    const int i0 = 8 * n + 2 * j;
    if constexpr (QT == 10) {
      const float d = half_at(bp + 80), dmin = half_at(bp + 82);
      const int c0 = bp[i0], c1 = bp[i0 + 1];
      return d * ((float)(c0 & 15) * s0 + (float)(c1 & 15) * s1) -
             dmin * ((float)(c0 >> 4) * x0 + (float)(c1 >> 4) * x1);
    } else {
      const uint8_t* sc = bp + 96;
      auto scale = [&](int i) {
        const int lo = i < 8 ? (sc[i] & 15) : (sc[i - 8] >> 4);
        return (float)((lo | (((sc[8 + (i & 3)] >> (2 * (i >> 2))) & 3) << 4)) - 32);
      };
      return half_at(bp + 108) * (scale(i0) * s0 + scale(i0 + 1) * s1);
    }
  } else if constexpr (QT == 13) {
    // Q5_K sub s: elements 32s + l, nibble s & 1 of qs[32(s/2) + l], bit s of
    // qh[l] as bit 4, scale / min s as Q4_K.
    int scv, mnv;
    scale_min_k4(bp + 4, sub, scv, mnv);
    const uint8_t* q = bp + 48 + 32 * (sub >> 1);
    const int sh = 4 * (sub & 1);
    float xv[32];
    load_x32<V4>(xb + 32 * sub, xv);
    float sq = 0.f, sx = 0.f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const int v = ((q[l] >> sh) & 15) | (((bp[16 + l] >> sub) & 1) << 4);
      sq += (float)v * xv[l];
      sx += xv[l];
    }
    return half_at(bp) * (float)scv * sq - half_at(bp + 2) * (float)mnv * sx;
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

// ---------------------------------------------------------------------------
// Direct kernel: no LDS.  Each wave computes R rows; lanes own fixed element
// groups of a block (LPB lanes per block, 64 / LPB blocks per wave step), so
// the x values a lane loads serve all R rows.  The decode is VALU-bound (a
// wave64 VALU op takes 4 cycles of a SIMD), so the formats are laid out to
// spend few ops per weight: per-block scale work is amortised over 16-32
// weights per lane, nibbles and bytes go to float with v_cvt_f32_ubyte*, and
// every row is a buffer resource (SGPRs) so the R rows share one 32-bit
// offset per load.  Q8_0 and Q6_K blocks start at 2-byte offsets: their
// fields are read as the dwords covering them and re-aligned with
// v_alignbyte (only dwords holding a field's bytes are read).
//
// Per format: LPB lanes per block, QKB elements per block, BB bytes, NX
// float4 of x per lane per block, NS partial sums of x per lane per block.
template <int QT>
struct QD;
template <>
struct QD<1> { static constexpr int LPB = 1, QKB = 8, BB = 16, NX = 2, NS = 0; };    // 8 halfs
template <>
struct QD<8> { static constexpr int LPB = 4, QKB = 32, BB = 34, NX = 2, NS = 1; };   // 8 int8
template <>
struct QD<6> { static constexpr int LPB = 4, QKB = 32, BB = 22, NX = 2, NS = 1; };   // 8 x 5 bit
template <>
struct QD<7> { static constexpr int LPB = 4, QKB = 32, BB = 24, NX = 2, NS = 1; };   // 8 x 5 bit
template <>
struct QD<20> { static constexpr int LPB = 4, QKB = 32, BB = 18, NX = 2, NS = 1; };  // 8 levels
template <>
struct QD<10> { static constexpr int LPB = 16, QKB = 256, BB = 84, NX = 4, NS = 4; };  // 16 x 2 bit
template <>
struct QD<11> { static constexpr int LPB = 16, QKB = 256, BB = 110, NX = 4, NS = 4; }; // 16 x 3 bit
template <>
struct QD<12> { static constexpr int LPB = 8, QKB = 256, BB = 144, NX = 8, NS = 2; };  // 32 nibbles
template <>
struct QD<13> { static constexpr int LPB = 8, QKB = 256, BB = 176, NX = 8, NS = 2; };  // 32 x 5 bit
template <>
struct QD<14> { static constexpr int LPB = 16, QKB = 256, BB = 210, NX = 4, NS = 4; }; // 16 x 6 bit

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int QT>
struct QRaw;
template <>
struct QRaw<1> { u32x4 h; };
template <>
struct QRaw<8> { u32x2 p; uint32_t q, d; };
template <>
struct QRaw<6> { uint32_t d, h0, h1, q0, q1; };
template <>
struct QRaw<7> { uint32_t dm0, dm1, h0, h1, q0, q1; };
template <>
struct QRaw<20> { uint32_t d, q0, q1; };
template <>
struct QRaw<10> { uint32_t q, dd; u32x2 sc; };
template <>
struct QRaw<11> { uint32_t q0, q1, h0, h1, s0, s1, s2, s3, d; };
template <>
struct QRaw<12> { u32x4 hdr, q; };
template <>
struct QRaw<13> { u32x4 hdr, q, h; };
template <>
struct QRaw<14> { uint32_t a0, a1, b0, b1, h0, h1; u32x2 s; uint32_t s2, d; };

typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Buffer resource over [base, base + bytes): raw byte addressing (stride 0),
// dword data format; a dword load that ends past `bytes` returns 0.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t bl32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off & ~3u, 0, 0);
}
__device__ __forceinline__ u32x2 bl64(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off & ~3u, 0, 0);
}
__device__ __forceinline__ u32x4 bl128(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t al(uint32_t hi, uint32_t lo, uint32_t ps) {
  return __builtin_amdgcn_alignbyte(hi, lo, ps);
}

// Element offsets (multiples of 4) within the block of lane j's x float4s.
template <int QT>
__device__ __forceinline__ int x_off(int j, int k) {
  if constexpr (QT == 1) return 4 * k;
  else if constexpr (QT == 8) return 8 * j + 4 * k;
  else if constexpr (QT == 6 || QT == 7 || QT == 20) return 16 * k + 4 * j;  // lo / hi nibbles
  else if constexpr (QT == 10 || QT == 11)  // 2-bit plane k of qs dword (n, g, l0)
    return 128 * (j >> 3) + 32 * k + 16 * ((j >> 2) & 1) + 4 * (j & 3);
  else if constexpr (QT == 12 || QT == 13)  // sub 2c: k < 4, sub 2c+1: k >= 4; 16 of each
    return 64 * (j >> 1) + 32 * (k >> 2) + 16 * (j & 1) + 4 * (k & 3);
  else return 128 * (j >> 3) + 32 * k + 4 * (j & 7);
}

// off: the block's first byte relative to the (dword-aligned) resource base.
template <int QT>
__device__ __forceinline__ void load_raw(rsrc_t rs, uint32_t off, int j, QRaw<QT>& r) {
  if constexpr (QT == 1) {
    r.h = bl128(rs, off);
  } else if constexpr (QT == 8) {
    const uint32_t a = off + 2 + 8 * j;
    r.p = bl64(rs, a);
    r.q = bl32(rs, a + 7);
    r.d = bl32(rs, off);
  } else if constexpr (QT == 6) {  // fp16 d, qh[4] at 2, qs[16] at 6
    r.d = bl32(rs, off);
    r.h0 = bl32(rs, off + 2);
    r.h1 = bl32(rs, off + 5);
    r.q0 = bl32(rs, off + 6 + 4 * j);
    r.q1 = bl32(rs, off + 9 + 4 * j);
  } else if constexpr (QT == 7) {  // fp16 d, fp16 m, qh[4] at 4, qs[16] at 8
    r.dm0 = bl32(rs, off);
    r.dm1 = bl32(rs, off + 3);
    r.h0 = bl32(rs, off + 4);
    r.h1 = bl32(rs, off + 7);
    r.q0 = bl32(rs, off + 8 + 4 * j);
    r.q1 = bl32(rs, off + 11 + 4 * j);
  } else if constexpr (QT == 20) {  // fp16 d, qs[16] at 2
    r.d = bl32(rs, off);
    r.q0 = bl32(rs, off + 2 + 4 * j);
    r.q1 = bl32(rs, off + 5 + 4 * j);
  } else if constexpr (QT == 10) {  // scales[16], qs[64] at 16, d, dmin at 80
    const uint32_t n = j >> 3, t = j & 7;  // t = 4g + l0/4
    r.q = bl32(rs, off + 16 + 32 * n + 4 * t);
    r.sc = bl64(rs, off + 8 * n);
    r.dd = bl32(rs, off + 80);
  } else if constexpr (QT == 11) {  // hmask[32], qs[64] at 32, scales[12] at 96, d at 108
    const uint32_t n = j >> 3, t = j & 7;
    r.q0 = bl32(rs, off + 32 + 32 * n + 4 * t);
    r.q1 = bl32(rs, off + 35 + 32 * n + 4 * t);
    r.h0 = bl32(rs, off + 4 * t);
    r.h1 = bl32(rs, off + 3 + 4 * t);
    r.s0 = bl32(rs, off + 96);
    r.s1 = bl32(rs, off + 100);
    r.s2 = bl32(rs, off + 104);
    r.s3 = bl32(rs, off + 107);
    r.d = bl32(rs, off + 108);
  } else if constexpr (QT == 12) {
    r.hdr = bl128(rs, off);
    r.q = bl128(rs, off + 16 + 32 * (j >> 1) + 16 * (j & 1));
  } else if constexpr (QT == 13) {
    r.hdr = bl128(rs, off);
    r.h = bl128(rs, off + 16 + 16 * (j & 1));
    r.q = bl128(rs, off + 48 + 32 * (j >> 1) + 16 * (j & 1));
  } else {
    const uint32_t n = j >> 3, l0 = 4 * (j & 7);
    r.a0 = bl32(rs, off + 64 * n + l0);
    r.a1 = bl32(rs, off + 64 * n + l0 + 3);
    r.b0 = bl32(rs, off + 64 * n + 32 + l0);
    r.b1 = bl32(rs, off + 64 * n + 32 + l0 + 3);
    r.h0 = bl32(rs, off + 128 + 32 * n + l0);
    r.h1 = bl32(rs, off + 128 + 32 * n + l0 + 3);
    r.s = bl64(rs, off + 192 + 8 * n);
    r.s2 = bl32(rs, off + 192 + 8 * n + 7);
    r.d = bl32(rs, off + 208);
  }
}

// Byte n of v as a float, one v_cvt_f32_ubyteN (written out: after a nibble
// mask the compiler otherwise narrows the extract to v_bfe + ubyte0, two ops).
#define HL_CVT_UBYTE(N)                                                   \
  __device__ __forceinline__ float cvt_ubyte##N(uint32_t v) {             \
    float r;                                                              \
    asm("v_cvt_f32_ubyte" #N " %0, %1" : "=v"(r) : "v"(v));               \
    return r;                                                             \
  }
HL_CVT_UBYTE(0)
HL_CVT_UBYTE(1)
HL_CVT_UBYTE(2)
HL_CVT_UBYTE(3)
#undef HL_CVT_UBYTE

// acc + sum of the 4 unsigned bytes of q times x.
__device__ __forceinline__ float fma4u(uint32_t q, const f32x4& x, float acc) {
  acc = fmaf(cvt_ubyte0(q), x.x, acc);
  acc = fmaf(cvt_ubyte1(q), x.y, acc);
  acc = fmaf(cvt_ubyte2(q), x.z, acc);
  return fmaf(cvt_ubyte3(q), x.w, acc);
}
__device__ __forceinline__ float hsum4(const f32x4& x) { return (x.x + x.y) + (x.z + x.w); }

// Per-step sums of x the formats subtract (offset-coded quants, Q4_K mins).
template <int QT>
__device__ __forceinline__ void x_sums(const f32x4* xv, float* xs) {
  if constexpr (QT == 8 || QT == 6 || QT == 7 || QT == 20) {
    xs[0] = hsum4(xv[0]) + hsum4(xv[1]);
  } else if constexpr (QT == 12 || QT == 13) {
    xs[0] = (hsum4(xv[0]) + hsum4(xv[1])) + (hsum4(xv[2]) + hsum4(xv[3]));
    xs[1] = (hsum4(xv[4]) + hsum4(xv[5])) + (hsum4(xv[6]) + hsum4(xv[7]));
  } else if constexpr (QT == 14 || QT == 10 || QT == 11) {
#pragma unroll
    for (int k = 0; k < 4; ++k) xs[k] = hsum4(xv[k]);
  }
}

// Q4_K / Q5_K 6-bit scales and mins of sub-blocks 2c and 2c+1: bytes
// 2(c&1), 2(c&1)+1 of 16-bit pairs built branch-free from the scale dwords
// Y = bytes 0-3, Z = 4-7, W = 8-11 (getScaleMinK4, quant.nim:235-242).
__device__ __forceinline__ void k4_pair(const u32x4& hdr, int c, float& sc0, float& sc1, float& mn0,
                                        float& mn1) {
  const uint32_t sh = 16 * (c & 1);
  const uint32_t Y = hdr.y >> sh, Z = hdr.z >> sh, W = hdr.w >> sh;
  const bool lo = c < 2;
  const uint32_t m1 = lo ? 0x3F3Fu : 0x0F0Fu, m2 = lo ? 0u : 0x3030u;
  const uint32_t SC = ((lo ? Y : W) & m1) | ((Y >> 2) & m2);
  const uint32_t MN = ((lo ? Z : (W >> 4)) & m1) | ((Z >> 2) & m2);
  sc0 = (float)(SC & 255u);
  sc1 = (float)((SC >> 8) & 255u);
  mn0 = (float)(MN & 255u);
  mn1 = (float)((MN >> 8) & 255u);
}

// ps: the block's first byte within its dword (0 or 2 for Q8_0 / Q6_K).
template <int QT>
__device__ __forceinline__ float compute_raw(const QRaw<QT>& r, int j, uint32_t ps, const f32x4* xv,
                                             const float* xs) {
  if constexpr (QT == 1) {
    const uint32_t h[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4& x = xv[i >> 1];
      const float a = f16_bits_to_f32((uint16_t)(h[i] & 0xFFFFu));
      const float b = f16_bits_to_f32((uint16_t)(h[i] >> 16));
      s = fmaf(a, (i & 1) ? x.z : x.x, s);
      s = fmaf(b, (i & 1) ? x.w : x.y, s);
    }
    return s;
  } else if constexpr (QT == 8) {
    // int8 q as the unsigned byte q ^ 0x80 = q + 128: sum((q+128) x) - 128 sum(x).
    const uint32_t sb = (ps + 2) & 3;  // the quants start 2 bytes after the block
    const uint32_t q0 = al(r.p.y, r.p.x, sb) ^ 0x80808080u, q1 = al(r.q, r.p.y, sb) ^ 0x80808080u;
    const float d = f16_bits_to_f32((uint16_t)((r.d >> (8 * ps)) & 0xFFFFu));
    return d * (fma4u(q1, xv[1], fma4u(q0, xv[0], 0.f)) - 128.f * xs[0]);
  } else if constexpr (QT == 6 || QT == 7 || QT == 20) {
    // Lane j: elements 4j..4j+3 (low nibbles of qs[4j..4j+3]) and
    // 16+4j..16+4j+3 (their high nibbles).  Fields sit at 2-byte offsets:
    // each is re-aligned by the block's own phase plus its offset.
    constexpr uint32_t QSO = QT == 6 ? 6 : QT == 7 ? 8 : 2;
    const uint32_t q = al(r.q1, r.q0, (ps + QSO) & 3);
    const uint32_t lo4 = q & 0x0F0F0F0Fu, hi4 = (q >> 4) & 0x0F0F0F0Fu;
    if constexpr (QT == 20) {
      const float d = f16_bits_to_f32((uint16_t)((r.d >> (8 * ps)) & 0xFFFFu));
      // levels as signed bytes, summed as unsigned (v ^ 0x80) minus 128 sum(x)
      const uint32_t a = iq4nl_levels4(lo4) ^ 0x80808080u, b = iq4nl_levels4(hi4) ^ 0x80808080u;
      return d * (fma4u(b, xv[1], fma4u(a, xv[0], 0.f)) - 128.f * xs[0]);
    } else {
      // bits 4j..4j+3 (low nibbles) and 16+4j.. (high) of qh into bit 4 of
      // each byte: b * 0x204081 moves bit i of a nibble to bit 8i.
      constexpr uint32_t QHO = QT == 6 ? 2 : 4;
      const uint32_t qh = al(r.h1, r.h0, (ps + QHO) & 3);
      const uint32_t bl = (qh >> (4 * j)) & 15u, bh = (qh >> (16 + 4 * j)) & 15u;
      const uint32_t u0 = lo4 | (((bl * 0x00204081u) & 0x01010101u) << 4);
      const uint32_t u1 = hi4 | (((bh * 0x00204081u) & 0x01010101u) << 4);
      const float dot = fma4u(u1, xv[1], fma4u(u0, xv[0], 0.f));
      if constexpr (QT == 6) {
        const float d = f16_bits_to_f32((uint16_t)((r.d >> (8 * ps)) & 0xFFFFu));
        return d * (dot - 16.f * xs[0]);
      } else {
        const uint32_t dm = al(r.dm1, r.dm0, ps);
        const float d = f16_bits_to_f32((uint16_t)(dm & 0xFFFFu));
        const float m = f16_bits_to_f32((uint16_t)(dm >> 16));
        return fmaf(d, dot, m * xs[0]);
      }
    }
  } else if constexpr (QT == 10 || QT == 11) {
    // Lane j = 8n + 4g + l0/4: elements 128n + 32k + 16g + l0..l0+3 for the
    // four 2-bit planes k of one qs dword; scale 8n + 2k + g per plane.
    const int n = j >> 3, g = (j >> 2) & 1;
    float acc = 0.f;
    if constexpr (QT == 10) {
      const float d = f16_bits_to_f32((uint16_t)(r.dd & 0xFFFFu));
      const float dmin = f16_bits_to_f32((uint16_t)(r.dd >> 16));
      float dsum = 0.f, msum = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t sb = ((k < 2 ? r.sc.x : r.sc.y) >> (8 * (2 * (k & 1) + g))) & 255u;
        dsum = fmaf((float)(sb & 15u), fma4u((r.q >> (2 * k)) & 0x03030303u, xv[k], 0.f), dsum);
        msum = fmaf((float)(sb >> 4), xs[k], msum);
      }
      acc = d * dsum - dmin * msum;
    } else {
      // value (q | h << 2) - 4 with h the hmask bit 4n + k; 6-bit scales:
      // low 4 bits at bits 4n of byte 2k + g, high 2 bits at bits
      // 2(2n + k/2) of byte 8 + 2(k&1) + g.
      const uint32_t q = al(r.q1, r.q0, ps), hm = al(r.h1, r.h0, ps);  // fields at 32 and 0
      const uint32_t S0 = al(r.s1, r.s0, ps), S1 = al(r.s2, r.s1, ps), S2 = al(r.s3, r.s2, ps);
      const float d = f16_bits_to_f32((uint16_t)((r.d >> (8 * ps)) & 0xFFFFu));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t u = ((q >> (2 * k)) & 0x03030303u) | (((hm >> (4 * n + k)) & 0x01010101u) << 2);
        const uint32_t lo = (((k < 2 ? S0 : S1) >> (8 * (2 * (k & 1) + g))) >> (4 * n)) & 15u;
        const uint32_t hi = (S2 >> (8 * (2 * (k & 1) + g) + 2 * (2 * n + (k >> 1)))) & 3u;
        const float sc = (float)(int)((lo | (hi << 4)) - 32u);
        acc = fmaf(sc, fma4u(u, xv[k], -4.f * xs[k]), acc);
      }
      acc *= d;
    }
    return acc;
  } else if constexpr (QT == 12 || QT == 13) {
    // Sub-blocks 2c (low nibbles) and 2c+1 (high nibbles); Q5_K adds bits
    // 2c / 2c+1 of qh[l] as bit 4.
    const int c = j >> 1;
    float sc0, sc1, mn0, mn1;
    k4_pair(r.hdr, c, sc0, sc1, mn0, mn1);
    const float d = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xFFFFu));
    const float dmin = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16));
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float slo = 0.f, shi = 0.f;
    if constexpr (QT == 12) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        slo = fma4u(q[m] & 0x0F0F0F0Fu, xv[m], slo);
        shi = fma4u(q[m] & 0xF0F0F0F0u, xv[4 + m], shi);  // 16 x nibble
      }
      shi *= 0.0625f;
    } else {
      const uint32_t h[4] = {r.h.x, r.h.y, r.h.z, r.h.w};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t hl = ((h[m] >> (2 * c)) & 0x01010101u) << 4;
        const uint32_t hh = ((h[m] >> (2 * c + 1)) & 0x01010101u) << 4;
        slo = fma4u((q[m] & 0x0F0F0F0Fu) | hl, xv[m], slo);
        shi = fma4u(((q[m] >> 4) & 0x0F0F0F0Fu) | hh, xv[4 + m], shi);
      }
    }
    return d * fmaf(sc0, slo, sc1 * shi) - dmin * fmaf(mn0, xs[0], mn1 * xs[1]);
  } else {
    const uint32_t qa = al(r.a1, r.a0, ps), qb = al(r.b1, r.b0, ps), qh = al(r.h1, r.h0, ps);
    const uint32_t slo = al(r.s.y, r.s.x, ps), shi = al(r.s2, r.s.y, ps);
    const float d = f16_bits_to_f32((uint16_t)((r.d >> (8 * ps)) & 0xFFFFu));
    const uint32_t hb = 8 * ((j & 7) >> 2);  // second scale of a 32-group for l >= 16
    const uint32_t u0 = (qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
    const uint32_t u1 = (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
    const uint32_t u2 = ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
    const uint32_t u3 = ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
    const float s0 = (float)(int8_t)((slo >> hb) & 255u);
    const float s1 = (float)(int8_t)((slo >> (16 + hb)) & 255u);
    const float s2 = (float)(int8_t)((shi >> hb) & 255u);
    const float s3 = (float)(int8_t)((shi >> (16 + hb)) & 255u);
    const float t0 = fma4u(u0, xv[0], -32.f * xs[0]);
    const float t1 = fma4u(u1, xv[1], -32.f * xs[1]);
    const float t2 = fma4u(u2, xv[2], -32.f * xs[2]);
    const float t3 = fma4u(u3, xv[3], -32.f * xs[3]);
    return d * fmaf(s0, t0, fmaf(s1, t1, fmaf(s2, t2, s3 * t3)));
  }
}

// KS waves (1, 2 or 4) split a row group's blocks (wave s of the group takes
// steps s, s + KS, ...) and merge through LDS; a workgroup holds 4 / KS
// row groups.  PAIR (R = 2): the group's two rows are row m of w and row m
// of w2, sharing the x registers; PAIR 1 stores silu(a) * b to y (fused
// gate / up / SiLU), PAIR 2 stores a to y and b to y2 (fused K / V).
// PAIR 3 (R = 2): the Q, K and V projections of one x in one launch: the
// first ceil(M / 2) groups are row pairs of w (M rows) into y, the next M2
// groups row m of w2 and of w3 into y2 and y3 (a wave-uniform choice of
// pointers; the arithmetic is the same code, so the results are those of
// the separate launches).
template <int QT, int R, int KS, int PAIR = 0>
__global__ __launch_bounds__(256) void quant_direct_kernel(const uint8_t* __restrict__ w,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y, int M, int K,
                                                           const uint8_t* __restrict__ w2,
                                                           float* __restrict__ y2,
                                                           const uint8_t* __restrict__ w3 = nullptr,
                                                           float* __restrict__ y3 = nullptr, int M2 = 0) {
  static_assert(PAIR == 0 || R == 2, "pairs are two rows");
  using F = QD<QT>;
  constexpr int BPI = 64 / F::LPB;
  __shared__ float part[4][R];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gi = blockIdx.x * (4 / KS) + wave / KS;  // row group
  const int gq = (M + 1) / 2;                        // PAIR 3: groups of the first matrix
  const bool qpart = PAIR != 3 || gi < gq;           // wave-uniform
  const int row0 = PAIR == 3 ? (qpart ? 2 * gi : gi - gq) : gi * (PAIR ? 1 : R);
  const int s0 = wave % KS;
  if (KS == 1 && (PAIR == 3 ? gi >= gq + M2 : row0 >= M)) return;  // no barrier below for KS == 1
  const int j = lane % F::LPB, bl = lane / F::LPB;
  const int nb = K / F::QKB;
  const uint32_t rowbytes = (uint32_t)nb * F::BB;
  const int iters = (nb + BPI - 1) / BPI;
  // One buffer resource per row, based at the dword holding its first byte.
  rsrc_t rs[R];
  uint32_t ps[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint8_t* rp;
    if (PAIR == 3 && !qpart) rp = (r == 0 ? w2 : w3) + (size_t)min(row0, M2 - 1) * rowbytes;
    else if (PAIR == 1 || PAIR == 2) rp = (r == 0 ? w : w2) + (size_t)min(row0, M - 1) * rowbytes;
    else rp = w + (size_t)min(row0 + r, M - 1) * rowbytes;
    ps[r] = (uint32_t)((uintptr_t)rp & 3);
    // Whole dwords: the range check drops a dword that ends past the size.
    rs[r] = make_rsrc(rp - ps[r], (rowbytes + ps[r] + 3) & ~3u);
  }
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;

  // Two register sets used in turn (a copy between them would wait for the
  // loads in flight): the next step's loads are issued before this step's
  // math.
  QRaw<QT> ra[R], rb[R];
  f32x4 xa[F::NX], xb[F::NX];
  auto load = [&](int it, QRaw<QT>* raw, f32x4* xv) {
    const int b = min(it * BPI + bl, nb - 1);
    const float* xp = x + (size_t)b * F::QKB;
#pragma unroll
    for (int k = 0; k < F::NX; ++k) xv[k] = *(const f32x4*)(xp + x_off<QT>(j, k));
#pragma unroll
    for (int r = 0; r < R; ++r) load_raw<QT>(rs[r], ps[r] + (uint32_t)b * F::BB, j, raw[r]);
  };
  auto compute = [&](int it, const QRaw<QT>* raw, const f32x4* xv) {
    const bool valid = it * BPI + bl < nb;
    const uint32_t b = (uint32_t)min(it * BPI + bl, nb - 1);
    float xs[F::NS > 0 ? F::NS : 1];
    x_sums<QT>(xv, xs);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = compute_raw<QT>(raw[r], j, (ps[r] + b * F::BB) & 3, xv, xs);
      acc[r] += valid ? v : 0.f;
    }
  };
  // Steps of this wave (wave-uniform: the look-ahead branch is scalar).
  const int nsteps = __builtin_amdgcn_readfirstlane(s0 < iters ? (iters - s0 + KS - 1) / KS : 0);
  if (nsteps > 0) load(s0, ra, xa);
  int p = 0;
  for (; p + 1 < nsteps; p += 2) {
    const int it = s0 + p * KS;
    load(it + KS, rb, xb);
    compute(it, ra, xa);
    if (p + 2 < nsteps) load(it + 2 * KS, ra, xa);
    compute(it + KS, rb, xb);
  }
  if (p < nsteps) compute(s0 + p * KS, ra, xa);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = acc[r];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o, 64);
    acc[r] = a;
  }
  auto store = [&](const float* t) {  // lane 0 of the group's first wave
    if constexpr (PAIR == 1) {
      if (row0 < M) y[row0] = t[0] * (1.0f / (1.0f + expf(-t[0]))) * t[1];  // gpuSiluMul
    } else if constexpr (PAIR == 2) {
      if (row0 < M) {
        y[row0] = t[0];
        y2[row0] = t[1];
      }
    } else if constexpr (PAIR == 3) {
      if (!qpart) {
        if (row0 < M2) {
          y2[row0] = t[0];
          y3[row0] = t[1];
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (row0 + r < M) y[row0 + r] = t[r];
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < M) y[row0 + r] = t[r];
    }
  };
  if (KS == 1) {
    if (lane == 0) store(acc);
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) part[wave][r] = acc[r];
  }
  __syncthreads();
  if (s0 == 0 && lane == 0) {
    float t[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      t[r] = 0.f;
#pragma unroll
      for (int i = 0; i < KS; ++i) t[r] += part[wave + i][r];
    }
    store(t);
  }
}

// ---------------------------------------------------------------------------
// Q4_K on MFMA (v_mfma_f32_16x16x32_f16): the products go to the matrix core,
// the VALU only unpacks nibbles.
//
// A step of a wave is 2 weight rows x 8 consecutive blocks (4096 weights):
// each load instruction reads 1152 contiguous bytes of each of the two rows.
// (The same bytes read as one block of each of 16 rows stream at ~3 TB/s.)
// The 16 MFMA columns n = 8 r + b are block b of row r; the 16 MFMA rows
// i = 2 b + c are part c of block b's x:
//   B[k][n] = quant at k of column n's block times its sub-block scale, as an
//             f16 bit pattern: q sc 2^-24 (<= 945 2^-24, exact; the low nibble
//             is one AND, the high nibble (16 q) is scaled by sc / 16),
//   A[i][k] = x of block b at k as x 2^s = h + m 2^-11 (two f16, 22
//             significant bits; s per block puts its largest |x| in
//             [2^13, 2^14)),
// so C[2b][n] + 2^-11 C[2b + 1][n] with b = n % 8 is the sum of sc q x over
// column n's block (exact products, fp32 accumulation); the rest of C is not
// used.  Lane 16 t + n holds quants group t of column n's block (sub-blocks
// 2t and 2t + 1: bytes 32 t..32 t + 31; MFMA j < 4 takes the low nibbles of
// bytes 8 j..8 j + 7, in k order 0,2,1,3,4,6,5,7, MFMA 4 + j the high ones),
// and C[2b..2b+1][n] lands in lane 16 (b / 2) + n, registers 2 (b % 2) and
// 2 (b % 2) + 1: that lane adds d 2^(24 - s) (C[2b] + 2^-11 C[2b+1]), and every
// lane subtracts dmin (mn0 X0 + mn1 X1) for its two sub-blocks (X: sums of
// x; getScaleMinK4 and dequantRowQ4K, quant.nim:235-277).
//
// Workgroups are persistent (about two per CU): x is converted once per
// workgroup into LDS in the A register layout (a wave keeps the 32 VGPRs of
// its 8-block group for all its steps).  The groups of a row go to different
// waves, the row pairs of the workgroup to the rest; partial sums meet in LDS.
// ---------------------------------------------------------------------------
constexpr int kQ4gA = 8 * 64 * 16;  // A of one 8-block group: [mfma 8][lane 64] x 16 B
constexpr int kQ4gX = 8 * 8 * 4;    // sub-block sums of x: [block 8][sub-block 8] floats
constexpr int kQ4gF = 8 * 4;        // 2^(24 - s) per block
constexpr int kQ4gBytes = kQ4gA + kQ4gX + kQ4gF;
constexpr int kQ4MaxGroups = 16;    // K <= 32768 (a workgroup of at most 16 waves)

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));

// Buffer resource over [base, base + bytes) (raw bytes; an access past
// `bytes` reads zeros), for the buffer-load builtins.  The base goes through
// readfirstlane: a resource the compiler cannot prove wave-uniform makes it
// wrap every load in a waterfall loop behind a full vmcnt(0) wait, which
// drains the prefetched loads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  const uintptr_t b = (uintptr_t)base;
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b) |
                     ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)u, 0, (int)bytes, 0x00020000);
}

// Lane l reads lane dpp(l) of v (within rows of 16 lanes).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Sum over the wave's 8-lane groups {16 t + 8 h + e : e < 8, t < 4} for each
// h: DPP within rows of 16 lanes, then the four rows.
__device__ __forceinline__ float half_row_sum(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// NORM: x is first replaced by rmsnorm(x + res) * nrm over its K values
// (gpuResidualRmsnorm, naive.nim:2845-2882, folded into the x prologue:
// every workgroup adds and reduces the whole vector; workgroup 0 also stores
// x + res to xsum, which no workgroup of this launch reads).  One x chunk
// per thread: K <= 8192.
template <int PAIR, bool NORM = false>
__global__ __launch_bounds__(1024) void q4k_mfma_kernel(const uint8_t* __restrict__ w,
                                                        const float* __restrict__ x,
                                                        float* __restrict__ y, int M, int K,
                                                        const uint8_t* __restrict__ w2,
                                                        float* __restrict__ y2, int rows_wg,
                                                        const float* __restrict__ res = nullptr,
                                                        const float* __restrict__ nrm = nullptr,
                                                        float* __restrict__ xsum = nullptr,
                                                        float eps = 0.f) {
  extern __shared__ __align__(16) char lds[];
  constexpr int NP = PAIR ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int nb = K / 256, ng = (nb + 7) / 8;
  float* part = (float*)(lds + ng * kQ4gBytes);  // [NP][ng][rows_wg]

  const int nstream = nw / ng;  // waves per group; the rest only meet the barriers
  const int g = wave % ng, st = wave / ng;
  const int n = lane & 15, t = lane >> 4, b8 = n & 7, rr = n >> 3;
  const int row0 = blockIdx.x * rows_wg;
  const int nrows = min(rows_wg, M - row0), npairs = (nrows + 1) / 2;
  const uint32_t rowbytes = (uint32_t)nb * 144u;
  const uint32_t oob = (uint32_t)nrows * rowbytes;  // past the workgroup's rows
  // Lane part of the weight offsets (a block past nb: beyond the range) and
  // the step's row pair as a uniform offset (a step past the last: beyond
  // the range; such loads return zeros without touching memory and a zero
  // step adds nothing).
  const uint32_t vb = 8 * g + b8 < nb ? (uint32_t)rr * rowbytes + (uint32_t)(8 * g + b8) * 144u : oob;
  const uint32_t vq = vb + 16 + 32 * t;
  const __amdgpu_buffer_rsrc_t rsw0 = buf_rsrc(w + (size_t)row0 * rowbytes, oob),
                               rsw1 = buf_rsrc((PAIR ? w2 : w) + (size_t)row0 * rowbytes, oob);
  struct Raw {
    u32x4 hdr, q0, q1;
  };
  // Step k: row pair st + (k / NP) nstream of matrix k % NP, three buffer
  // loads (the compiler counts them for its waits).  Scheduling barriers
  // around each step's loads keep the next steps' loads where they are
  // issued, three steps ahead of their math, instead of below it.
  const int nsteps = __builtin_amdgcn_readfirstlane(
      st < nstream && st < npairs ? ((npairs - st + nstream - 1) / nstream) * NP : 0);
  auto load = [&](int k, Raw& r) {
    const int pm = PAIR ? (k & 1) : 0, q = st + (PAIR ? k >> 1 : k) * nstream;
    const uint32_t so = __builtin_amdgcn_readfirstlane(k < nsteps ? (uint32_t)(2 * q) * rowbytes : oob);
    const __amdgpu_buffer_rsrc_t rs = PAIR && pm ? rsw1 : rsw0;  // a uniform select of SGPR resources
    __builtin_amdgcn_sched_barrier(0);
    r.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vb, (int)so, 0);
    r.q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vq, (int)so, 0);
    r.q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vq + 16, (int)so, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // x -> LDS.  Chunk c = x[8c, 8c + 8) is one A register of block bk = c / 32
  // (group bk / 8, block bk % 8 in it), quants group t, MFMA 4 h + j
  // (8 c mod 256 = 64 t + 32 h + 8 j); a block's 32 chunks are 32 consecutive
  // threads.  Blocks past nb are written as zeros (their quants load as
  // zeros too).
  const __amdgpu_buffer_rsrc_t xdesc = buf_rsrc(x, (uint32_t)K * 4u);
  auto x_chunk = [&](int c, f32x4& v0, f32x4& v1) {
    v0 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xdesc, 32 * c, 0, 0));
    v1 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xdesc, 32 * c + 16, 0, 0));
  };
  auto convert = [&](int c, const f32x4& v0, const f32x4& v1) {
    const int bk = c >> 5, cb = c & 31;
    float am = fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                     fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w))));
    am = fmaxf(am, dpp_f32<kDppXor1>(am));
    am = fmaxf(am, dpp_f32<kDppXor2>(am));
    am = fmaxf(am, dpp_f32<kDppHalfMirror>(am));
    am = fmaxf(am, dpp_f32<kDppMirror>(am));     // 16 chunks
    am = fmaxf(am, __shfl_xor(am, 16, 64));       // the block's 32
    float sum = (hsum4(v0) + hsum4(v1));
    sum += dpp_f32<kDppXor1>(sum);
    sum += dpp_f32<kDppXor2>(sum);                // the sub-block's 4 chunks
    // am = f 2^e, f in [0.5, 1): am 2^(14 - e) in [2^13, 2^14).  (am = 0, inf,
    // nan: e = 0.)
    const int s = min(max(14 - __builtin_amdgcn_frexp_expf(am), -100), 140);
    const float xs[8] = {ldexpf(v0.x, s), ldexpf(v0.z, s), ldexpf(v0.y, s), ldexpf(v0.w, s),
                         ldexpf(v1.x, s), ldexpf(v1.z, s), ldexpf(v1.y, s), ldexpf(v1.w, s)};
    f16x8 hv, mv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hv[e] = (_Float16)xs[e];
      mv[e] = (_Float16)((xs[e] - (float)hv[e]) * 2048.f);
    }
    if (c >= ng * 256) return;  // threads past the last chunk
    const int bb = bk & 7, ct = cb >> 3, mf = cb & 7;  // mf = 4 h + j
    char* gb = lds + (bk >> 3) * kQ4gBytes;
    *(f16x8*)(gb + (mf * 64 + 16 * ct + 2 * bb) * 16) = hv;
    *(f16x8*)(gb + (mf * 64 + 16 * ct + 2 * bb + 1) * 16) = mv;
    if ((cb & 3) == 0) ((float*)(gb + kQ4gA))[bb * 8 + (cb >> 2)] = sum;  // sub-block 2t + h
    if (cb == 0) ((float*)(gb + kQ4gA + kQ4gX))[bb] = ldexpf(1.0f, 24 - s);
  };
  // All of this thread's x chunks (at most 4: a workgroup has at least one
  // wave per group; NORM: one, with its res and nrm chunks), then the first
  // three steps' weights, which stay in flight while x is converted.
  constexpr int XC = NORM ? 1 : 4;
  f32x4 xv[XC][2];
#pragma unroll
  for (int i = 0; i < XC; ++i) x_chunk(threadIdx.x + i * blockDim.x, xv[i][0], xv[i][1]);
  [[maybe_unused]] f32x4 rv[2], nv[2];
  if constexpr (NORM) {
    const __amdgpu_buffer_rsrc_t rdesc = buf_rsrc(res, (uint32_t)K * 4u), ndesc = buf_rsrc(nrm, (uint32_t)K * 4u);
    const int o = 32 * (int)threadIdx.x;
    rv[0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rdesc, o, 0, 0));
    rv[1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rdesc, o + 16, 0, 0));
    nv[0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ndesc, o, 0, 0));
    nv[1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ndesc, o + 16, 0, 0));
  }
  Raw ra, rb, rc;
  load(0, ra);  // the loads' scheduling barriers keep x's loads ahead of these
  load(1, rb);
  load(2, rc);
  if constexpr (NORM) {
    // Chunks past K load as zeros and add nothing to the sum of squares.
    const f32x4 v0 = xv[0][0] + rv[0], v1 = xv[0][1] + rv[1];
    float ss = (v0.x * v0.x + v0.y * v0.y) + (v0.z * v0.z + v0.w * v0.w) +
               ((v1.x * v1.x + v1.y * v1.y) + (v1.z * v1.z + v1.w * v1.w));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    float* red = (float*)(lds + ng * kQ4gBytes) + NP * ng * rows_wg;
    if (lane == 0) red[wave] = ss;
    if (blockIdx.x == 0 && (int)threadIdx.x < K / 8) {
      *(f32x4*)(xsum + 8 * threadIdx.x) = v0;
      *(f32x4*)(xsum + 8 * threadIdx.x + 4) = v1;
    }
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    const float inv = 1.0f / sqrtf(t / (float)K + eps);
    xv[0][0] = f32x4{v0.x * inv * nv[0].x, v0.y * inv * nv[0].y, v0.z * inv * nv[0].z, v0.w * inv * nv[0].w};
    xv[0][1] = f32x4{v1.x * inv * nv[1].x, v1.y * inv * nv[1].y, v1.z * inv * nv[1].z, v1.w * inv * nv[1].w};
  }
#pragma unroll
  for (int i = 0; i < XC; ++i)
    if ((int)(threadIdx.x & ~63u) + i * (int)blockDim.x < ng * 256)  // wave-uniform
      convert(threadIdx.x + i * blockDim.x, xv[i][0], xv[i][1]);
  __syncthreads();

  if (st < nstream) {
    const char* gb = lds + g * kQ4gBytes;
    f16x8 av[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) av[m] = *(const f16x8*)(gb + (m * 64 + lane) * 16);
    const float2 X = *(const float2*)(gb + kQ4gA + (b8 * 8 + 2 * t) * 4);
    const float fblk = ((const float*)(gb + kQ4gA + kQ4gX))[b8];
    const bool diag = (b8 >> 1) == t;
    const bool odd = b8 & 1;

    auto compute = [&](int k, const Raw& r) {
      float sc0, sc1, mn0, mn1;
      k4_pair(r.hdr, t, sc0, sc1, mn0, mn1);
      const float d = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xFFFFu));
      const float dmin = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16));
      const h2v s0 = {(_Float16)sc0, (_Float16)sc0};
      const h2v s1 = {(_Float16)(sc1 * 0.0625f), (_Float16)(sc1 * 0.0625f)};
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t d0 = j < 2 ? r.q0[2 * j] : r.q1[2 * j - 4];
        const uint32_t d1 = j < 2 ? r.q0[2 * j + 1] : r.q1[2 * j - 3];
        const uint32_t e0 = d0 >> 8, e1 = d1 >> 8;
        const uint32_t lq[4] = {d0 & 0x000F000Fu, e0 & 0x000F000Fu, d1 & 0x000F000Fu, e1 & 0x000F000Fu};
        const uint32_t hq[4] = {d0 & 0x00F000F0u, e0 & 0x00F000F0u, d1 & 0x00F000F0u, e1 & 0x00F000F0u};
        u32x4 bl, bh;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          bl[u] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, lq[u]) * s0);
          bh[u] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, hq[u]) * s1);
        }
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[j], __builtin_bit_cast(f16x8, bl), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[4 + j], __builtin_bit_cast(f16x8, bh), c, 0, 0, 0);
      }
      const float vh = odd ? c[2] : c[0], vm = odd ? c[3] : c[1];
      float a = -dmin * fmaf(mn0, X.x, mn1 * X.y);
      if (diag) a = fmaf(d * fblk, fmaf(vm, 0x1p-11f, vh), a);
      a = half_row_sum(a);  // lanes n < 8: row 0 of the pair, n >= 8: row 1
      const int pm = PAIR ? (k & 1) : 0, q = st + (PAIR ? k >> 1 : k) * nstream;
      if ((lane & 7) == 0 && lane < 16 && 2 * q + rr < nrows)
        part[(pm * ng + g) * rows_wg + 2 * q + rr] = a;
    };
    // Three steps in flight: a step's registers are reloaded with the step
    // three ahead right after its math.  Loads and waits are unconditional,
    // so the counts hold on every path (loads past the last step read
    // nothing).
    for (int k = 0; k < nsteps; k += 3) {
      compute(k, ra);
      load(k + 3, ra);
      if (k + 1 < nsteps) compute(k + 1, rb);
      load(k + 4, rb);
      if (k + 2 < nsteps) compute(k + 2, rc);
      load(k + 5, rc);
    }
  }
  __syncthreads();
  for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
    float a = 0.f, b = 0.f;
    for (int gg = 0; gg < ng; ++gg) {
      a += part[gg * rows_wg + r];
      if (PAIR) b += part[(ng + gg) * rows_wg + r];
    }
    if constexpr (PAIR == 0) {
      y[row0 + r] = a;
    } else if constexpr (PAIR == 1) {
      y[row0 + r] = a * (1.0f / (1.0f + expf(-a))) * b;  // gpuSiluMul
    } else {
      y[row0 + r] = a;
      y2[row0 + r] = b;
    }
  }
}

// The MFMA kernel pays for its x prologue (~2 us of latency before the
// first product) on matrices of 2^25 weights and more: 14336 x 4096 10.8 us
// against 15.7, 4096 x 14336 14.2 against 17.0, but 4096 x 4096 8.3 against
// 6.6 (kernel durations).  A fused pair streams both matrices behind one x
// prologue, so pairs count 2 M rows: two 8192 x 2048 matrices (the
// Llama-3.2-1B gate/up) move to the matrix cores, with the FFN norm folded
// in (Llama-3.2-1B decode 0.73 -> 0.65 ms/token as a graph).
constexpr size_t kQ4MaxLds = 160 * 1024;  // LDS per CU (gfx950)

bool q4k_mfma_pays(int M, int K) {
  return K <= 256 * 8 * kQ4MaxGroups && (long long)M * K >= (1LL << 25);
}

// Workgroup: one wave per 8-block group times row-pair streams, with at
// least one thread per x chunk when 16 waves allow it; as many workgroups
// as are resident at once (LDS and 16 waves per CU) share the row pairs.
template <int PAIR, bool NORM = false>
bool launch_q4k_mfma(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t stream,
                     const uint8_t* w2 = nullptr, float* y2 = nullptr, const float* res = nullptr,
                     const float* nrm = nullptr, float* xsum = nullptr, float eps = 0.f) {
  const int nb = K / 256, ng = (nb + 7) / 8;
  // Waves: 4 streams of row pairs per 8-block group up to 4 groups, 2 up to
  // 8 groups (16 waves at most): at K = 14336 one workgroup per CU with two
  // streams converts x once per CU instead of twice (4096 x 14336: 13.7 ->
  // 12.9 us).
  const int nw = ng <= 4 ? 4 * ng : (ng <= 8 ? 2 * ng : ng);
  const size_t a_bytes = (size_t)ng * kQ4gBytes;
  const int per_cu = std::max(1, std::min<int>(16 / nw, (int)((160 * 1024) / (a_bytes + 4096))));
  const int pairs = (M + 1) / 2;
  const int wgs_target = per_cu * cu_count();
  int pairs_wg = (pairs + wgs_target - 1) / wgs_target;
  // The per-row partial sums grow with the rows per workgroup: past 160 KiB
  // of LDS the rows go to more workgroups instead (they queue behind the
  // resident ones).
  const size_t fixed = (size_t)ng * kQ4gBytes + (NORM ? 16 * 4 : 0);
  const size_t per_row = (size_t)(PAIR ? 2 : 1) * ng * 4;
  const int max_pairs = (int)((kQ4MaxLds - fixed) / per_row / 2);
  pairs_wg = std::max(1, std::min(pairs_wg, max_pairs));
  const int rows = 2 * pairs_wg;
  const size_t shm = fixed + per_row * rows;
  // The attribute is set once per instantiation; without it only 64 KiB of
  // dynamic LDS may be asked for, and a larger case goes to the direct kernel.
  static const hipError_t attr = hipFuncSetAttribute((const void*)q4k_mfma_kernel<PAIR, NORM>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)kQ4MaxLds);
  if (shm > kQ4MaxLds || (attr != hipSuccess && shm > 64 * 1024)) {
    (void)hipGetLastError();  // the failed attribute call's error is not this launch's
    return false;
  }
  hipLaunchKernelGGL((q4k_mfma_kernel<PAIR, NORM>), dim3((M + rows - 1) / rows), dim3(64 * nw), shm, stream, w,
                     x, y, M, K, w2, y2, rows, res, nrm, xsum, eps);
  return true;
}

template <int QT, int R, int KS, int PAIR = 0>
void launch_direct(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t stream,
                   const uint8_t* w2 = nullptr, float* y2 = nullptr, const uint8_t* w3 = nullptr,
                   float* y3 = nullptr, int M2 = 0) {
  const int groups = PAIR == 3 ? (M + 1) / 2 + M2 : PAIR ? M : (M + R - 1) / R;
  const int grid = (groups + 4 / KS - 1) / (4 / KS);
  hipLaunchKernelGGL((quant_direct_kernel<QT, R, KS, PAIR>), dim3(grid), dim3(256), 0, stream, w, x, y,
                     M, K, w2, y2, w3, y3, M2);
}

template <int QT, int KS>
void launch_direct_r(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t stream) {
  constexpr bool r4 = QT != 12 && QT != 13 && QT != 14;  // the K-quants at four rows: ~200+ VGPRs
  if (r4 && M >= 8192) launch_direct<QT, 4, KS>(w, x, y, M, K, stream);
  else if (M >= 2048) launch_direct<QT, 2, KS>(w, x, y, M, K, stream);
  else launch_direct<QT, 1, KS>(w, x, y, M, K, stream);
}

template <int QT>
void launch_direct_plan(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t stream) {
  // Split a row's blocks over four waves when each gets a step: more waves
  // and loads in flight for decode-sized M.  (A two-way split of 2-3 steps
  // measured slower than none: Q4_K 4096x4096 5.5 -> 7.2 us.)
  if constexpr (QT == 12) {
    if (q4k_mfma_pays(M, K) && launch_q4k_mfma<0>(w, x, y, M, K, stream)) return;
  }
  const int iters = (K / QD<QT>::QKB + 64 / QD<QT>::LPB - 1) / (64 / QD<QT>::LPB);
  // Tall matrices (output heads: 128256 rows) keep each row in one wave:
  // with 64K+ row pairs the grid is full anyway, and a wave's four steps
  // pipeline their loads (Q6_K 128256x4096 184 -> 130 us, Q5_0 112 -> 102 us).
  // Four to seven steps per row go to two waves, two or more steps each
  // (against four waves: Q6_K 14336x4096 20.2 -> 14.9 us, Q2_K 18.2 -> 13.8,
  // Q4_K 2048x8192 6.1 -> 4.9, Q5_K 4096x14336 15.5 -> 14.5).
  if (M >= 65536 || iters < 4) launch_direct_r<QT, 1>(w, x, y, M, K, stream);
  else if (iters < 8) launch_direct_r<QT, 2>(w, x, y, M, K, stream);
  else launch_direct_r<QT, 4>(w, x, y, M, K, stream);
}

// Two matrices of one type at once (PAIR 1 or 2), when the direct kernel
// takes their pointers; false: the caller runs them separately.
template <int QT, int PAIR>
bool launch_pair_qt(const uint8_t* w, const uint8_t* w2, const float* x, float* y, float* y2, int M,
                    int K, hipStream_t stream) {
  const long long rowbytes = (long long)(K / QD<QT>::QKB) * QD<QT>::BB;
  const uintptr_t a = (uintptr_t)w | (uintptr_t)w2;
  const bool ok = ((uintptr_t)x & 15) == 0 && rowbytes < (1LL << 31) && K % QD<QT>::QKB == 0 &&
                  (QT == 1 ? (a & 15) == 0 : (QT == 12 || QT == 13) ? (a & 15) == 0
                   : QT == 10 ? (a & 3) == 0 : (a & 1) == 0);
  if (!ok) return false;
  if constexpr (QT == 12) {
    if (q4k_mfma_pays(2 * M, K) && launch_q4k_mfma<PAIR>(w, x, y, M, K, stream, w2, y2)) return true;
  }
  const int iters = (K / QD<QT>::QKB + 64 / QD<QT>::LPB - 1) / (64 / QD<QT>::LPB);
  // The block split follows the single-matrix rule (two waves for four to
  // seven steps: Q6_K gate/up 14336x4096 43.0 -> 32.0 us, Q3_K 43.3 -> 30.0,
  // Q2_K 30.4 -> 24.1).
  if (iters >= 8) launch_direct<QT, 2, 4, PAIR>(w, x, y, M, K, stream, w2, y2);
  else if (iters >= 4) launch_direct<QT, 2, 2, PAIR>(w, x, y, M, K, stream, w2, y2);
  else launch_direct<QT, 2, 1, PAIR>(w, x, y, M, K, stream, w2, y2);
  return true;
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

// F16 rows of any length (the reference's F16 GEMV, naive.nim:1342-1366,
// takes any wCols): one wave per row, lanes stride the columns.  Used only
// when K is not a multiple of 32; other F16 shapes take the kernels above.
__global__ __launch_bounds__(256) void f16_gemv_any_kernel(const uint16_t* __restrict__ w,
                                                           const float* __restrict__ x,
                                                           float* __restrict__ y, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* wr = w + (size_t)row * K;
  float acc = 0.f;
  for (int c = lane; c < K; c += 64) acc = fmaf(f16_bits_to_f32(wr[c]), x[c], acc);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) y[row] = acc;
}

template <int QT>
void launch_qt(const uint8_t* w, const float* x, float* y, int M, int K, hipStream_t stream) {
  const long long rowbytes = (long long)(K / QFmt<QT>::QK) * QFmt<QT>::BYTES;
  const bool aligned = rowbytes % 4 == 0 && ((uintptr_t)w & 3) == 0;
  const bool v4 = ((uintptr_t)x & 15) == 0;
  // Direct kernel when x is 16-byte aligned and the blocks are as aligned as
  // the format allows (F16 rows of whole 8-half groups on 16 bytes, Q4_K on
  // 16, Q8_0 / Q6_K on 2).
  const uintptr_t wa = (uintptr_t)w;
  constexpr bool has_direct = true;
  const bool direct = has_direct && v4 && rowbytes < (1LL << 31) &&
                      (QT == 1 ? (K % 8 == 0 && (wa & 15) == 0)
                       : (QT == 12 || QT == 13) ? (wa & 15) == 0
                       : QT == 10 ? (wa & 3) == 0 : (wa & 1) == 0);  // Q2_K: 84-byte blocks, no phase
  if constexpr (has_direct) {
    if (direct) {
      launch_direct_plan<QT>(w, x, y, M, K, stream);
      return;
    }
  }
  if (M >= 2048) launch_q<QT, 1>(w, x, y, M, K, aligned, v4, stream);
  else launch_q<QT, 4>(w, x, y, M, K, aligned, v4, stream);
}

}  // namespace

int quant_block_elems(int qtype) {
  switch (qtype) {
    case HL_GGML_F16: case HL_GGML_Q5_0: case HL_GGML_Q5_1: case HL_GGML_Q8_0: case HL_GGML_IQ4_NL:
      return 32;
    case HL_GGML_Q2_K: case HL_GGML_Q3_K: case HL_GGML_Q4_K: case HL_GGML_Q5_K: case HL_GGML_Q6_K:
      return 256;
    default: return 0;
  }
}

long long quant_row_bytes(int qtype, int K) {
  switch (qtype) {
    case HL_GGML_F16: return 2LL * K;
    case HL_GGML_Q5_0: return (long long)(K / 32) * 22;
    case HL_GGML_Q5_1: return (long long)(K / 32) * 24;
    case HL_GGML_Q8_0: return (long long)(K / 32) * 34;
    case HL_GGML_IQ4_NL: return (long long)(K / 32) * 18;
    case HL_GGML_Q2_K: return (long long)(K / 256) * 84;
    case HL_GGML_Q3_K: return (long long)(K / 256) * 110;
    case HL_GGML_Q4_K: return (long long)(K / 256) * 144;
    case HL_GGML_Q5_K: return (long long)(K / 256) * 176;
    case HL_GGML_Q6_K: return (long long)(K / 256) * 210;
    default: return 0;
  }
}

// y = silu(W_gate x) * (W_up x) (PAIR 1) or y = W_a x, y2 = W_b x (PAIR 2)
// in one launch for two matrices of one GGUF type; returns false when the
// pointers or the type do not allow it (the caller then runs them apart).
bool linear_quant_pair_launch(int pair, float* y, float* y2, const float* x, const void* wa,
                              const void* wb, int K, int M, int qtype, hipStream_t stream) {
  const uint8_t *a = (const uint8_t*)wa, *b = (const uint8_t*)wb;
#define HL_PAIR(QT)                                                        \
  return pair == 1 ? launch_pair_qt<QT, 1>(a, b, x, y, nullptr, M, K, stream) \
                   : launch_pair_qt<QT, 2>(a, b, x, y, y2, M, K, stream)
  switch (qtype) {
    case HL_GGML_F16: if (K % 8) return false; HL_PAIR(1);
    case HL_GGML_Q5_0: HL_PAIR(6);
    case HL_GGML_Q5_1: HL_PAIR(7);
    case HL_GGML_Q8_0: HL_PAIR(8);
    case HL_GGML_Q2_K: HL_PAIR(10);
    case HL_GGML_Q3_K: HL_PAIR(11);
    case HL_GGML_Q4_K: HL_PAIR(12);
    case HL_GGML_Q5_K: HL_PAIR(13);
    case HL_GGML_Q6_K: HL_PAIR(14);
    case HL_GGML_IQ4_NL: HL_PAIR(20);
    default: return false;
  }
#undef HL_PAIR
}

// The Q, K and V projections of one x in one launch (three matrices of one
// GGUF type, each K columns; Q has Mq rows, K and V have Mkv): the direct
// kernel's PAIR 3 mode.  Returns false when the pointers, the type or the
// shapes do not allow it (Q4_K matrices that the matrix-core kernel takes,
// for instance); the caller then runs the projections apart.
template <int QT>
bool launch_qkv_qt(const uint8_t* wq, const uint8_t* wk, const uint8_t* wv, const float* x, float* yq,
                   float* yk, float* yv, int Mq, int Mkv, int K, hipStream_t stream) {
  const long long rowbytes = (long long)(K / QD<QT>::QKB) * QD<QT>::BB;
  const uintptr_t a = (uintptr_t)wq | (uintptr_t)wk | (uintptr_t)wv;
  const bool ok = ((uintptr_t)x & 15) == 0 && rowbytes < (1LL << 31) && K % QD<QT>::QKB == 0 &&
                  (QT == 1 ? (a & 15) == 0 : (QT == 12 || QT == 13) ? (a & 15) == 0
                   : QT == 10 ? (a & 3) == 0 : (a & 1) == 0);
  if (!ok) return false;
  if constexpr (QT == 12) {
    if (q4k_mfma_pays(Mq, K) || q4k_mfma_pays(Mkv, K)) return false;
  }
  const int iters = (K / QD<QT>::QKB + 64 / QD<QT>::LPB - 1) / (64 / QD<QT>::LPB);
  if (iters >= 8) launch_direct<QT, 2, 4, 3>(wq, x, yq, Mq, K, stream, wk, yk, wv, yv, Mkv);
  else if (iters >= 4) launch_direct<QT, 2, 2, 3>(wq, x, yq, Mq, K, stream, wk, yk, wv, yv, Mkv);
  else launch_direct<QT, 2, 1, 3>(wq, x, yq, Mq, K, stream, wk, yk, wv, yv, Mkv);
  return true;
}

// Residual + RMSNorm folded into the fused gate/up/SiLU GEMV (Q4_K on the
// matrix cores, K <= 8192): xsum = x + res; y = silu(G n) * (U n) with
// n = rmsnorm(xsum) * nrm.  false: not this kernel's case (the caller runs
// the norm and the pair separately).
bool linear_quant_gate_up_norm_launch(float* y, float* xsum, const float* x, const float* res, const float* nrm,
                                      float eps, const void* wg, const void* wu, int K, int M, int qtype,
                                      hipStream_t stream) {
  const uintptr_t v = (uintptr_t)x | (uintptr_t)res | (uintptr_t)nrm | (uintptr_t)xsum;
  const uintptr_t a = (uintptr_t)wg | (uintptr_t)wu;
  if (qtype != HL_GGML_Q4_K || M <= 0 || K <= 0 || K % 256 || K > 8192 || (v & 15) || (a & 15) ||
      !q4k_mfma_pays(2 * M, K))
    return false;
  return launch_q4k_mfma<1, true>((const uint8_t*)wg, x, y, M, K, stream, (const uint8_t*)wu, nullptr, res, nrm,
                                  xsum, eps);
}

bool linear_quant_qkv_launch(float* yq, float* yk, float* yv, const float* x, const void* wq, const void* wk,
                             const void* wv, int K, int Mq, int Mkv, int qtype, hipStream_t stream) {
  const uint8_t *a = (const uint8_t*)wq, *b = (const uint8_t*)wk, *c = (const uint8_t*)wv;
  if (Mq <= 0 || Mkv <= 0) return false;
#define HL_QKV(QT) return launch_qkv_qt<QT>(a, b, c, x, yq, yk, yv, Mq, Mkv, K, stream)
  switch (qtype) {
    case HL_GGML_F16: if (K % 8) return false; HL_QKV(1);
    case HL_GGML_Q5_0: HL_QKV(6);
    case HL_GGML_Q5_1: HL_QKV(7);
    case HL_GGML_Q8_0: HL_QKV(8);
    case HL_GGML_Q2_K: HL_QKV(10);
    case HL_GGML_Q3_K: HL_QKV(11);
    case HL_GGML_Q4_K: HL_QKV(12);
    case HL_GGML_Q5_K: HL_QKV(13);
    case HL_GGML_Q6_K: HL_QKV(14);
    case HL_GGML_IQ4_NL: HL_QKV(20);
    default: return false;
  }
#undef HL_QKV
}

hipError_t linear_quant_launch(float* y, const float* x, const void* w, int K, int M, int qtype,
                               hipStream_t stream) {
  const uint8_t* wb = (const uint8_t*)w;
  switch (qtype) {
    case HL_GGML_F16:
      if (K % 32 == 0) launch_qt<1>(wb, x, y, M, K, stream);
      else hipLaunchKernelGGL(f16_gemv_any_kernel, dim3((M + 3) / 4), dim3(256), 0, stream,
                              (const uint16_t*)w, x, y, M, K);
      break;
    case HL_GGML_Q5_0: launch_qt<6>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q5_1: launch_qt<7>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q8_0: launch_qt<8>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q2_K: launch_qt<10>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q3_K: launch_qt<11>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q4_K: launch_qt<12>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q5_K: launch_qt<13>(wb, x, y, M, K, stream); break;
    case HL_GGML_Q6_K: launch_qt<14>(wb, x, y, M, K, stream); break;
    case HL_GGML_IQ4_NL: launch_qt<20>(wb, x, y, M, K, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace hl
